"""GPU parity of the single-pass top-p path (rows with top-k off and 0 < top_p < 1, and greedy
rows asking for logprobs) against the CPU oracle.

The path keeps the elements above a sampled threshold as candidates and sums the rest with the
hardware exp2, then decides top-p exactly when the approximation's error bound allows and hands
the row to the exact multi-pass path when it does not.  Either way the results must equal the
oracle's bit for bit (tokens, flags, survivor counts, logprob ids and ranks; logprob values
within rtol 1e-5).  The FLAG_STREAM_TOPP diagnostic bit says which path served a row; the
benchmark workloads must mostly take the single pass."""
import numpy as np
import pytest

from tests.common import assert_same, gpu_run, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu

STREAM = 0x200
GENERAL = 0x100
WIDE = 0x800


def _wl(x, T, p, k=0, mp=0.0, L=None, seed=0, dtype="f32"):
    B, V = x.shape
    rng = np.random.default_rng(1000 + seed)
    full = lambda v, dt: np.full(B, v, dt)  # noqa: E731
    Ta = np.asarray(T, np.float32) if np.ndim(T) else full(T, np.float32)
    pa = np.asarray(p, np.float32) if np.ndim(p) else full(p, np.float32)
    u = (rng.integers(1, 2 ** 24, size=(B, V)).astype(np.float32) * np.float32(2.0 ** -24))
    logits = W._bf16_bits(x) if dtype == "bf16" else x.astype(np.float32)
    return W.Workload("topp case", logits, dtype, Ta, full(k, np.int32), pa,
                      full(mp, np.float32), full(1.0, np.float32), full(0.0, np.float32),
                      full(0.0, np.float32), None, u, num_logprobs=L)


def _check(w, cuda, label, min_stream=None):
    ref = oracle_run(w)
    got = gpu_run(w, cuda)
    stream = int(((got["flags"] & STREAM) != 0).sum())
    general = int(((got["flags"] & GENERAL) != 0).sum())
    why = np.bincount((got["flags"] >> 16) & 0xFF, minlength=9)[1:]
    wide = int(((got["flags"] & WIDE) != 0).sum())
    print(f"{label}: {w.shape} stream rows {stream} (wide {wide}), multi-pass rows {general}, "
          f"fallback reasons {why.tolist()}", flush=True)
    assert_same(got, ref, label)
    if min_stream is not None:
        assert stream >= min_stream * w.shape[0], f"{label}: only {stream} rows took the single pass"
    return got


def test_c5_full_mostly_single_pass(cuda):
    w = W.config(5)
    _check(w, cuda, "C5 full", min_stream=0.9)


def test_c5_scaled_without_logprobs(cuda):
    w = W.config(5, scale=0.25)
    w.num_logprobs = None
    _check(w, cuda, "C5/4 no logprobs", min_stream=0.8)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("T", [0.3, 0.7, 1.0, 1.5])
def test_temperatures(cuda, dtype, T):
    rng = np.random.default_rng(int(T * 10) + (7 if dtype == "bf16" else 0))
    x = rng.normal(0, 3, (24, 50000)).astype(np.float32)
    x += W._zipf_bias(rng, 50000, 1.1)[None, :]
    p = rng.uniform(0.5, 0.98, 24).astype(np.float32)
    _check(_wl(x, T, p, seed=int(T * 10), dtype=dtype), cuda, f"T={T} {dtype}")


def test_nan_and_inf_entries(cuda):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (16, 30000)).astype(np.float32)
    x[:, ::7] = np.nan
    x[:, 3::11] = -np.inf
    x[5, :] = -np.inf
    x[5, 100] = 1.0
    _check(_wl(x, 0.9, 0.9, seed=3), cuda, "nan/inf")


def test_quantised_ties_at_the_boundary(cuda):
    rng = np.random.default_rng(4)
    x = (np.round(rng.normal(0, 3, (24, 40000)) * 2) / 2).astype(np.float32)
    p = np.linspace(0.3, 0.99, 24).astype(np.float32)
    _check(_wl(x, 1.0, p, seed=4), cuda, "ties")
    _check(_wl(x, 0.5, p, seed=5, dtype="bf16"), cuda, "ties bf16")


@pytest.mark.parametrize("mp", [0.01, 0.05, 0.3])
def test_min_p_with_top_p(cuda, mp):
    rng = np.random.default_rng(int(mp * 100))
    x = rng.normal(0, 3, (16, 60000)).astype(np.float32)
    _check(_wl(x, 1.2, 0.95, mp=mp, seed=6), cuda, f"min_p {mp}")


@pytest.mark.parametrize("V", [1, 7, 100, 1000, 6000])
def test_small_vocabularies(cuda, V):
    rng = np.random.default_rng(V)
    x = rng.normal(0, 2, (8, V)).astype(np.float32)
    _check(_wl(x, 0.8, 0.7, seed=V, L=min(V, 5)), cuda, f"V={V}")


@pytest.mark.parametrize("p", [1e-4, 0.01, 0.5, 0.999, 0.99999])
def test_top_p_extremes(cuda, p):
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, (12, 40000)).astype(np.float32)   # flat rows: huge nuclei near p = 1
    _check(_wl(x, 1.0, p, seed=11), cuda, f"p={p}")


@pytest.mark.parametrize("L", [0, 5, 64])
def test_greedy_rows_with_logprobs(cuda, L):
    rng = np.random.default_rng(20 + L)
    x = rng.normal(0, 3, (16, 70000)).astype(np.float32)
    x[3, [10, 500, 69999]] = 50.0    # tied maxima: the lowest index wins
    x[4, :] = 2.0                    # a constant row
    _check(_wl(x, 0.0, 1.0, seed=L, L=L), cuda, f"greedy L={L}")


@pytest.mark.parametrize("T", [1.0, 0.6])
def test_logprobs_with_sampling(cuda, T):
    rng = np.random.default_rng(int(T * 100))
    x = rng.normal(0, 3, (16, 80000)).astype(np.float32)
    x += W._zipf_bias(rng, 80000, 1.2)[None, :]
    _check(_wl(x, T, 0.9, seed=30, L=20), cuda, f"logprobs T={T}")


def test_mixed_batch_with_top_k_rows(cuda):
    """Top-p-only rows, top-k rows (single-pass kernel), greedy rows and logprobs together."""
    rng = np.random.default_rng(40)
    B, V = 32, 65536
    x = rng.normal(0, 4, (B, V)).astype(np.float32)
    T = rng.uniform(0.2, 1.4, B).astype(np.float32)
    T[::6] = 0.0
    p = rng.uniform(0.6, 0.99, B).astype(np.float32)
    w = _wl(x, T, p, seed=40)
    w.top_k[1::4] = 40
    _check(w, cuda, "mixed")
    w.num_logprobs = 8
    _check(w, cuda, "mixed + logprobs")


def test_strided_unaligned_rows(cuda):
    """Rows of a strided view whose starts are not 16-byte aligned (head and tail elements)."""
    import torch

    from oracle import sampler as O
    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(50)
    B, V, pad = 8, 30001, 3
    base = rng.normal(0, 3, (B, V + pad)).astype(np.float32)
    u = (rng.integers(1, 2 ** 24, size=(B, V)).astype(np.float32) * np.float32(2.0 ** -24))
    T = np.full(B, 0.8, np.float32)
    p = np.full(B, 0.9, np.float32)
    xt = torch.from_numpy(base).to(cuda)[:, 1:V + 1]
    res = ops.sample(xt, temperature=torch.from_numpy(T), top_p=torch.from_numpy(p),
                     uniforms=torch.from_numpy(u).to(cuda))
    torch.cuda.synchronize()
    x = np.ascontiguousarray(base[:, 1:V + 1])
    prm = O.make_params(B, T, np.zeros(B, np.int32), p, 0.0, 1.0, 0.0, 0.0)
    ref = O.sample(x, prm, u)
    assert np.array_equal(res.sampled.cpu().numpy(), ref["token"])
    assert np.array_equal(res.num_kept.cpu().numpy(), ref["n_kept"])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("L", [None, 3])
def test_wide_rows(cuda, dtype, L):
    """Nuclei far larger than the candidate buffers (flat rows, high temperature, p near 1): one
    exact pass over the logits and uniforms decides them; every fourth row also has a min-p
    that keeps survivors below the candidates, and with logprobs the sampled token is mostly
    not a candidate (its rank takes a pass of its own)."""
    rng = np.random.default_rng(60 + (L or 0) + (5 if dtype == "bf16" else 0))
    B, V = 16, 120000
    x = rng.normal(0, 1.5, (B, V)).astype(np.float32)
    T = rng.uniform(0.9, 1.6, B).astype(np.float32)
    p = rng.uniform(0.9, 0.999, B).astype(np.float32)
    w = _wl(x, T, p, seed=60, dtype=dtype, L=L)
    w.min_p[::4] = np.float32(0.001)
    got = _check(w, cuda, f"wide {dtype} L={L}")
    assert int(((got["flags"] & WIDE) != 0).sum()) >= B - 2


def test_boundary_bucket_sizes(cuda):
    """Boundary buckets (1/64 of a unit of y) of about 1000, 340, 100 and 20 members: values
    uniform over [-a, 0], V = 262144, p = 0.5.  For a = 4 and 12 the nucleus is far larger than
    the candidate buffers (wide rows: most members come from the pass over the logits); for
    a = 40 and 200 it lies among the candidates.  The members are sorted above 512, ranked by
    several threads per member from 65 to 512 and by one thread up to 64."""
    rng = np.random.default_rng(77)
    V = 262144
    spans = [4.0, 4.0, 12.0, 12.0, 40.0, 40.0, 200.0, 200.0]
    x = np.stack([-rng.uniform(0.0, a, V) for a in spans]).astype(np.float32)
    w = _wl(x, 1.0, 0.5, seed=77)
    got = _check(w, cuda, "boundary bucket sizes")
    assert int(((got["flags"][:4] & WIDE) != 0).sum()) == 4

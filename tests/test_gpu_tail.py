"""GPU parity of the single-pass kernel's finish at its boundaries.

Rows with k <= 64 are finished by one wave from the 65 largest candidates in key order; larger k
by the multi-wave finish; anything the single pass cannot settle exactly goes to the multi-pass
path.  These cases sit on each of those edges: k around 64, ties at the k-th value that run past
the 64th slot, greedy rows with more than 64 tied maxima, top-p <= 0 or tiny, min-p 1, rows with
fewer finite logits than k, and quantised logits where ties are everywhere.  Token ids, flags and
survivor counts must match the oracle bit for bit."""
import numpy as np
import pytest

from tests.cases import _wl
from tests.common import assert_same, gpu_run, oracle_run

pytestmark = pytest.mark.gpu


def _check(cuda, w):
    assert_same(gpu_run(w, cuda), oracle_run(w), w.name)


@pytest.mark.parametrize("V", [20000, 128256])
def test_k_around_one_wave(cuda, V):
    rng = np.random.default_rng(101)
    ks = np.array([1, 2, 31, 63, 64, 65, 100, 256] * 2, np.int32)
    B = ks.size
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    T = np.where(np.arange(B) % 8 == 7, 0.0, 0.7).astype(np.float32)  # a few greedy rows
    _check(cuda, _wl(f"k_around_64_V{V}", x, T, k=ks, p=0.9, seed=1))


@pytest.mark.parametrize("ntie,k", [(63, 40), (64, 40), (65, 40), (80, 50), (64, 64), (65, 64),
                                    (200, 10)])
def test_ties_at_kth_past_the_slots(cuda, ntie, k):
    """ntie copies of the row maximum: with ntie > 64 the top k (ties kept) has more members
    than one wave holds."""
    rng = np.random.default_rng(ntie * 7 + k)
    B, V = 6, 40000
    x = rng.normal(0, 1, (B, V)).astype(np.float32)
    for b in range(B):
        x[b, rng.choice(V, ntie, replace=False)] = 6.0
    _check(cuda, _wl(f"ties{ntie}_k{k}", x, 0.8, k=k, p=np.float32(0.5 + 0.1 * (k % 3)), seed=2))


def test_greedy_many_tied_maxima(cuda):
    rng = np.random.default_rng(7)
    B, V = 5, 60000
    x = rng.normal(0, 1, (B, V)).astype(np.float32)
    for b, n in enumerate([2, 64, 65, 300, 5000]):
        x[b, rng.choice(V, n, replace=False)] = 9.5
    _check(cuda, _wl("greedy_ties", x, 0.0, k=0, seed=3))
    _check(cuda, _wl("greedy_ties_k", x, 0.0, k=50, seed=3))


@pytest.mark.parametrize("p,mp", [(0.0, 0.0), (1e-7, 0.0), (0.3, 1.0), (0.999999, 0.0),
                                  (1.0, 0.2)])
def test_topp_minp_extremes(cuda, p, mp):
    rng = np.random.default_rng(int(p * 1000) + int(mp * 10))
    B, V = 8, 32000
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    _check(cuda, _wl(f"p{p}_mp{mp}", x, 1.3, k=np.array([1, 5, 20, 50, 64, 65, 90, 7], np.int32),
                     p=p, mp=mp, seed=4))


def test_fewer_finite_than_k(cuda):
    rng = np.random.default_rng(9)
    B, V = 4, 25000
    x = np.full((B, V), -np.inf, np.float32)
    for b, n in enumerate([1, 10, 49, 70]):
        x[b, rng.choice(V, n, replace=False)] = rng.normal(0, 2, n).astype(np.float32)
    _check(cuda, _wl("few_finite", x, 0.9, k=50, p=0.8, seed=5))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_quantised_logits(cuda, dtype):
    """Logits on a grid of 0.25 (about 40 distinct values): ties at every rank, including
    across the temperature division."""
    rng = np.random.default_rng(13)
    B, V = 12, 50000
    x = (np.round(rng.normal(0, 2, (B, V)) * 4) / 4).astype(np.float32)
    ks = np.array([3, 5, 50, 64, 65, 1] * 2, np.int32)
    T = np.array([0.7, 0.3, 1.0, 1.7, 0.55, 0.0] * 2, np.float32)
    if dtype == "bf16":
        from vllm_webgpu_amd.workloads import _bf16_bits
        w = _wl("quantised_bf16", _bf16_bits(x), T, k=ks, p=0.9, seed=6, dtype="bf16")
    else:
        w = _wl("quantised_f32", x, T, k=ks, p=0.9, seed=6)
    _check(cuda, w)


def test_small_k_with_penalties(cuda):
    rng = np.random.default_rng(17)
    B, V, H = 8, 70000, 300
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    # the history includes each row's largest logits, so the penalties reorder the top
    for b in range(B):
        hist[b, :20] = np.argsort(-x[b])[:20]
    w = _wl("small_k_penalties", x, np.array([0.7, 0.0] * 4, np.float32),
            k=np.array([50, 50, 64, 1, 10, 64, 65, 20], np.int32), p=0.9, mp=0.05,
            rep=1.3, pres=0.4, freq=0.2, hist=hist, seed=8)
    _check(cuda, w)


@pytest.mark.parametrize("k", [2, 10, 50, 64, 100])
def test_seed_above_kth(cuda, k):
    """Spikes packed into the first iteration (the seed's sample) push the seed above the row's
    k-th value: fewer than k candidates pass it, and the row must be finished exactly anyway."""
    rng = np.random.default_rng(200 + k)
    B, V = 4, 128256
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    for b in range(B):
        n = max(1, k - 1 - b)  # fewer spikes than k
        x[b, rng.choice(20000, n, replace=False)] = 40.0 + rng.random(n).astype(np.float32)
    _check(cuda, _wl(f"seed_high_k{k}", x, 0.9, k=k, p=0.95, seed=9))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_unaligned_strided_rows(cuda, dtype):
    """Rows of a strided view whose starts are not 16-byte aligned (odd offset and stride, odd
    V): the unaligned head and tail of every row go through the edge loads, on the single-pass
    path (k <= 64 and k > 64), greedy rows and the multi-pass path (top-k off)."""
    import torch

    from vllm_webgpu_amd import ops
    from vllm_webgpu_amd.workloads import _bf16_bits

    rng = np.random.default_rng(31)
    B, V, pad = 8, 50001, 6
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[:, 0] = 30.0 + np.arange(B)        # maxima in the unaligned head ...
    x[1::2, V - 1] = 60.0                # ... and in the tail of odd rows
    ks = np.array([50, 1, 64, 65, 0, 200, 5, 0], np.int32)
    T = np.array([0.8, 0.0, 1.1, 0.7, 0.9, 1.0, 0.0, 1.3], np.float32)
    w = _wl(f"strided_{dtype}", _bf16_bits(x) if dtype == "bf16" else x, T, k=ks, p=0.9, seed=12,
            dtype=dtype)
    ref = oracle_run(w)
    if dtype == "bf16":
        wide = np.zeros((B, V + pad), np.uint16)
        wide[:, 3:3 + V] = w.logits
        base = torch.from_numpy(wide.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        wide = np.zeros((B, V + pad), np.float32)
        wide[:, 3:3 + V] = w.logits
        base = torch.from_numpy(wide).to(cuda)
    logits = base[:, 3:3 + V]
    assert logits.stride(0) == V + pad and logits.data_ptr() % 16 != 0
    res = ops.sample(logits, temperature=torch.from_numpy(w.temperature),
                     top_k=torch.from_numpy(w.top_k), top_p=torch.from_numpy(w.top_p),
                     uniforms=torch.from_numpy(w.uniforms).to(cuda))
    torch.cuda.synchronize()
    gpu = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
               n_kept=res.num_kept.cpu().numpy())
    assert_same(gpu, ref, w.name)

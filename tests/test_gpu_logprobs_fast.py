"""GPU parity of raw logprobs on the single pass: launches that ask for logprobs no longer send
every top-k or greedy row to the multi-pass path.  The single pass keeps at least max(k, L)
candidates, sums exp(x - a) over the whole row while it streams, and finishes the top-L ids and
values, the sampled token's rank and the log-normaliser from the candidates.

Token ids, flags, survivor counts, logprob ids and ranks are compared bit for bit with the
oracle, logprob values at 1e-5 (fp32 logits)."""
import numpy as np
import pytest

from tests.cases import _wl
from tests.common import assert_same, gpu_run, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu

GENERAL = 0x100


def test_c3_full_with_20_logprobs_stays_on_the_single_pass(cuda):
    w = W.config(3)
    w.num_logprobs = 20
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), "C3 + 20 logprobs")
    n = int(((g["flags"] & GENERAL) != 0).sum())
    assert n == 0, f"{n} of 256 rows took the multi-pass path"


@pytest.mark.parametrize("L", [0, 1, 5, 20, 64])
def test_logprob_counts_and_mixed_rows(cuda, L):
    """Rows with k below and above L, greedy rows, top-p-only rows (the top-p path), k above 64
    (the 32-bit packing) and k = 256, in one launch."""
    rng = np.random.default_rng(200 + L)
    B, V = 40, 30000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    k = np.array([5, 1, 20, 50, 64, 65, 100, 256, 0, 3] * 4, np.int32)
    T = np.where(np.arange(B) % 7 == 0, 0.0, 0.8).astype(np.float32)
    p = np.where(k == 0, 0.9, 0.95).astype(np.float32)
    w = _wl(f"mixed L={L}", x, T, k=k, p=p, seed=L, L=L)
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), w.name)
    # (k = 256 rows leave the single pass at this V with or without logprobs: their seed pool
    # is too small, and unseeded they pack more than 1024 candidates)
    single = ((k > 0) & (k <= 100)) | (T == 0)
    assert not (g["flags"][single] & GENERAL).any()


def test_ties_at_the_lth_value_and_penalties(cuda):
    """Logits on a coarse grid (many ties at the L-th raw value: ids ascending within a tie)
    and penalties from a history (the candidates' processed keys differ from the raw ones the
    logprobs use)."""
    rng = np.random.default_rng(31)
    B, V = 32, 20000
    x = (np.round(rng.normal(0, 2, (B, V)) * 2) / 2).astype(np.float32)
    hist = rng.integers(0, V, (B, 300)).astype(np.int32)
    top = np.argsort(-x, axis=1, kind="stable")[:, :30].astype(np.int32)
    hist[:, :30] = top                                  # penalise the raw leaders
    w = _wl("grid ties + penalties", x, 0.9, k=40, p=0.9, rep=1.3, pres=0.5, freq=0.2, hist=hist,
            seed=32, L=20)
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), w.name)


def test_bf16_and_f16_with_logprobs(cuda):
    """Logprobs on the single pass for 16-bit logits (8 elements per 16-byte vector)."""
    rng = np.random.default_rng(41)
    B, V = 24, 50021  # odd V: unaligned tails
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    for dt in ("bf16", "f16"):
        w = _wl(f"{dt} logprobs", x, 0.7, k=50, p=0.9, seed=42, L=10)
        if dt == "bf16":
            u = x.view(np.uint32).astype(np.uint64)
            w.logits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        else:
            w.logits = x.astype(np.float16)
        w.dtype = dt
        g = gpu_run(w, cuda)
        assert_same(g, oracle_run(w), w.name)
        assert not (g["flags"] & GENERAL).any()


def test_extreme_rows_fall_back_exactly(cuda):
    """Rows the single pass hands on with logprobs: a spike far above the first iteration
    (the stream's sum overflows), NaN logits, -inf logits, fewer finite values than L."""
    rng = np.random.default_rng(51)
    B, V = 8, 40000
    x = rng.normal(0, 1, (B, V)).astype(np.float32)
    x[0, 39000] = 200.0            # 200 above the first iteration's maximum
    x[1, 123] = np.nan
    x[2, : V - 5] = -np.inf        # 5 finite values, L = 8
    x[3, ::2] = -np.inf
    w = _wl("extreme rows", x, 1.0, k=20, p=0.9, seed=52, L=8)
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), w.name)

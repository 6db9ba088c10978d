"""GPU parity of the fused logit soft cap (Gemma's final cap * tanh(x / cap), applied to the
logits before everything else) against the oracle, which caps each row first and then samples.

The single-pass kernel thresholds the raw logits and caps only its candidates; its exactness
check bounds the capped value of everything below a threshold (the fp32 tanh is not monotone,
so the bound carries a margin).  These cases cover that pass (k <= 64 and k > 64, greedy),
rows it hands to the multi-pass kernel (saturated ties at +cap, capped values too close to
settle, raising penalties, logprobs, no top-k), the processors, and bf16 logits.  Token ids,
flags and survivor counts must match the oracle bit for bit; logprob values within 1e-5."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import _wl
from tests.common import FLAG_MASK, assert_same, gpu_run, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu

GENERAL = 0x100


def _check(cuda, w, cap, L=None):
    g = gpu_run(w, cuda, num_logprobs=L, softcap=cap)
    assert_same(g, oracle_run(w, num_logprobs=L, softcap=cap), w.name)
    return g


@pytest.mark.parametrize("fn_range", [(-20.0, 20.0), (20.0, 3.0e38), (-3.0e38, -20.0)])
def test_softcap_bit_exact(cuda, fn_range):
    """The device's capped tanh gives the oracle's bits on every fp32 of the range."""
    from vllm_webgpu_amd import ops

    lo, hi = fn_range
    ref = O.check_softcap(lo, hi)
    h, c = ops.math_selftest(2, O.key(lo), O.key(hi))
    assert c == ref["count"]
    assert h == ref["hash"]


@pytest.mark.parametrize("V", [32000, 128256, 262144])
def test_single_pass_small_and_large_k(cuda, V):
    rng = np.random.default_rng(21)
    ks = np.array([50, 1, 20, 64, 65, 100, 256, 50] * 2, np.int32)
    B = ks.size
    x = (rng.standard_normal((B, V)) * 12.0).astype(np.float32)
    T = np.where(np.arange(B) % 8 == 7, 0.0, 0.7).astype(np.float32)
    g = _check(cuda, _wl(f"cap_k_V{V}", x, T, k=ks, p=0.9, seed=21), 30.0)
    # The capped single pass keeps raw values in its buffers and cannot cut them, so it needs
    # a seed threshold: at Gemma's vocabulary (262144) every k <= 256 gets one; with a small
    # vocabulary large k go to the multi-pass kernel.
    settled = ks <= 64 if V == 32000 else np.ones(B, bool)
    assert not np.any(g["flags"][settled] & GENERAL)


def test_headline_shape_with_cap(cuda):
    rng = np.random.default_rng(22)
    B, V = 64, 128256
    x = (rng.standard_normal((B, V)) * 8.0).astype(np.float32)
    hist = rng.integers(0, V, (B, 128)).astype(np.int32)
    w = _wl("cap_c3", x, 0.7, k=50, p=0.9, rep=1.1, pres=0.5, freq=0.3, hist=hist, seed=22)
    g = _check(cuda, w, 30.0)
    assert not np.any(g["flags"] & GENERAL)


def test_saturated_ties_at_cap(cuda):
    """Logits beyond 20 * cap all cap to exactly +cap: ties in capped space that are not ties
    in raw space.  Greedy takes the lowest index of them; top-k keeps them all."""
    rng = np.random.default_rng(23)
    B, V = 6, 50000
    x = (rng.standard_normal((B, V)) * 5.0).astype(np.float32)
    for b, n in enumerate([1, 3, 40, 64, 65, 300]):
        x[b, rng.choice(V, n, replace=False)] = rng.uniform(700.0, 5000.0, n).astype(np.float32)
    g = _check(cuda, _wl("cap_sat_greedy", x, 0.0, k=0, seed=23), 30.0)
    big = x >= 600.0
    first = np.array([np.nonzero(big[b])[0][0] for b in range(B)])
    assert np.array_equal(g["token"], first)
    g = _check(cuda, _wl("cap_sat_k", x, 0.8, k=np.array([1, 2, 50, 50, 64, 10], np.int32),
                         p=0.7, seed=24), 30.0)
    assert g["flags"][5] & GENERAL                 # 300 tied members: more than one wave holds


def test_values_too_close_to_settle(cuda):
    """Raw logits where the cap's tanh is within a few ulps of 1 (x / cap near 8): many
    distinct raw values share capped values, which the single pass must order exactly or
    leave to the multi-pass kernel."""
    rng = np.random.default_rng(25)
    B, V = 8, 40000
    x = (rng.standard_normal((B, V)) * 3.0).astype(np.float32)
    for b in range(B):
        n = 30 + 20 * b
        x[b, rng.choice(V, n, replace=False)] = rng.uniform(7.5 * 30, 9.0 * 30, n).astype(np.float32)
    T = np.array([0.7, 0.0] * 4, np.float32)
    _check(cuda, _wl("cap_close", x, T, k=50, p=0.95, seed=25), 30.0)


def test_general_path_rows(cuda):
    """No top-k with a history from id lists, top-k past the single pass, min-p, and a raising
    (negative) presence penalty: served by the multi-pass kernel with the cap on every logit."""
    rng = np.random.default_rng(26)
    B, V = 8, 60000
    x = (rng.standard_normal((B, V)) * 10.0).astype(np.float32)
    hist = rng.integers(0, V, (B, 200)).astype(np.int32)
    w = _wl("cap_general", x, np.array([0.7, 1.0, 0.0, 0.5, 1.3, 0.7, 0.9, 0.0], np.float32),
            k=np.array([0, 0, 0, 400, 1000, 0, 50, 20], np.int32),
            p=np.array([0.9, 0.5, 1.0, 0.9, 1.0, 0.3, 0.8, 1.0], np.float32),
            mp=np.array([0.0, 0.1, 0.0, 0.0, 0.05, 0.0, 0.0, 0.0], np.float32),
            rep=1.2, pres=np.array([0.0, 0.0, 0.0, 0.0, 0.0, 0.0, -0.5, -0.5], np.float32),
            freq=0.1, hist=hist, seed=26)
    _check(cuda, w, 25.0)


@pytest.mark.parametrize("L", [0, 5])
def test_logprobs_of_capped_logits(cuda, L):
    rng = np.random.default_rng(27 + L)
    B, V = 6, 32000
    x = (rng.standard_normal((B, V)) * 20.0).astype(np.float32)
    w = _wl("cap_lp", x, np.array([0.7, 0.0, 1.0, 0.7, 0.0, 1.1], np.float32), k=50, p=0.9, seed=27)
    _check(cuda, w, 30.0, L=L)


def test_penalties_on_the_top(cuda):
    """Penalties that only lower logits, on histories holding each row's largest logits: the
    single pass applies them to the capped values of its candidates; rows whose penalised
    candidates fall below its threshold are finished by the multi-pass kernel."""
    rng = np.random.default_rng(28)
    B, V, H = 8, 70000, 300
    x = (rng.standard_normal((B, V)) * 10.0).astype(np.float32)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    for b in range(B):
        hist[b, :20] = np.argsort(-x[b])[:20]
    w = _wl("cap_penalties", x, np.array([0.7, 0.0] * 4, np.float32),
            k=np.array([50, 50, 64, 1, 10, 64, 65, 20], np.int32), p=0.9, mp=0.05,
            rep=1.3, pres=0.4, freq=0.2, hist=hist, seed=28)
    _check(cuda, w, 30.0)


def test_bf16_logits(cuda):
    from vllm_webgpu_amd.workloads import _bf16_bits

    rng = np.random.default_rng(29)
    B, V = 12, 50000
    x = (rng.standard_normal((B, V)) * 15.0).astype(np.float32)
    ks = np.array([3, 50, 64, 65, 1, 0] * 2, np.int32)
    T = np.array([0.7, 0.3, 1.0, 1.7, 0.0, 0.9] * 2, np.float32)
    _check(cuda, _wl("cap_bf16", _bf16_bits(x), T, k=ks, p=0.9, seed=29, dtype="bf16"), 30.0)


@pytest.mark.parametrize("pos_bias", [False, True])
def test_processors_after_the_cap(cuda, pos_bias):
    """Bans and biases apply to the capped logits (the model's output)."""
    from tests.test_gpu_processors import _adjust, _run
    from vllm_webgpu_amd import workloads as W

    w = W.config(3, scale=0.05)
    rng = np.random.default_rng(31 + pos_bias)
    ids, vals = _adjust(rng, w.logits_f32(), 40, ban_top=3, pos_bias=pos_bias)
    _run(cuda, w, w.logits, ids, vals, softcap=30.0)
    B, V = w.shape
    allowed = rng.random((B, V)) < 0.5
    _run(cuda, w, w.logits, allowed=allowed, softcap=30.0)


def test_cap_off_is_unchanged(cuda):
    """logit_softcap None and 0 are the same launch as before the cap existed."""
    rng = np.random.default_rng(33)
    x = (rng.standard_normal((8, 20000)) * 4.0).astype(np.float32)
    w = _wl("cap_off", x, 0.8, k=40, p=0.9, seed=33)
    a = gpu_run(w, cuda)
    b = gpu_run(w, cuda, softcap=0.0)
    for key in ("token", "flags", "n_kept"):
        assert np.array_equal(a[key], b[key])
    assert np.array_equal(a["flags"] & FLAG_MASK, oracle_run(w)["flags"] & FLAG_MASK)


STREAM_TOPP = 0x200


@pytest.mark.parametrize("f16", [False, True])
def test_topp_rows_with_the_cap(cuda, f16):
    """Top-p rows without top-k under the cap (Gemma's sampling): the top-p stream caps every
    logit as it loads it (and its f16 store when asked), so the rows stay on it; T != 1, min-p,
    greedy rows with logprobs, 20 raw logprobs of the capped logits, saturated logits."""
    rng = np.random.default_rng(141)
    B, V = 48, 262144 // 4
    x = (rng.standard_normal((B, V)) * 10.0).astype(np.float32)
    x[::9, :50] = 400.0                                     # saturated at +cap
    T = np.where(np.arange(B) % 6 == 5, 0.0, np.where(np.arange(B) % 2 == 0, 1.0, 0.8)).astype(np.float32)
    mp = np.where(np.arange(B) % 4 == 1, 0.02, 0.0).astype(np.float32)
    w = _wl("cap_topp", x, T, k=0, p=0.95, mp=mp, seed=142, L=20)
    g = gpu_run(w, cuda, softcap=30.0, softcap_f16=f16)
    assert_same(g, oracle_run(w, softcap=30.0, softcap_f16=f16), w.name)
    on = (g["flags"] & STREAM_TOPP) != 0
    assert on.mean() > 0.9, f"{int((~on).sum())} of {B} rows left the top-p stream"


def test_topp_capped_flat_rows_take_the_passes(cuda):
    """Flat rows under the cap: the exact and wide passes cap each element as they load it,
    in chunks shared with other workgroups."""
    rng = np.random.default_rng(143)
    B, V = 40, 120000
    x = (rng.normal(0, 0.4, (B, V))).astype(np.float32)
    x[::5] *= 60.0
    w = _wl("cap flat", x, 0.9, k=0, p=0.97, seed=144)
    g = gpu_run(w, cuda, softcap=30.0)
    assert_same(g, oracle_run(w, softcap=30.0), w.name)
    assert (g["flags"] & STREAM_TOPP).all()
    assert (g["flags"] & (0x400 | 0x800)).any(), "no capped row took a further pass"


def test_c4_shape_with_the_cap(cuda):
    """C4 (512 x 262144 bf16, mixed rows) under Gemma's cap of 30 with the f16 store: (nearly)
    every row served by the single-pass paths."""
    w = W.config(4)
    g = gpu_run(w, cuda, softcap=30.0, softcap_f16=True)
    assert_same(g, oracle_run(w, softcap=30.0, softcap_f16=True), "C4 + cap")
    gen = (g["flags"] & GENERAL) != 0
    assert gen.mean() < 0.03, f"{int(gen.sum())} of 512 rows took the multi-pass path"

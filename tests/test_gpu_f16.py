"""GPU parity for float16 logits (the reference's f16 logits, sampled without a cast) and for
the soft cap whose output is stored in f16 (vllm_webgpu/shaders/gemma/logit_softcap.wgsl:28).

f16 values widen exactly to fp32, so the oracle samples the widened logits: token ids, flags
and survivor counts must match bit for bit, logprob values within 1e-5.  The device's
fp32 -> f16 -> fp32 rounding is checked against the oracle's on every fp32 of several ranges
(the oracle's rounding is itself pinned against numpy's float16 cast in
test_oracle_softcap.py)."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import _wl
from tests.common import assert_same, gpu_run, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu

STREAM = 0x200


@pytest.mark.parametrize("lo,hi", [(2.0 ** -27, 2.0 ** -13), (-2.0 ** -13, -2.0 ** -27),
                                   (0.5, 4.0), (-40.0, -20.0), (60000.0, 70000.0),
                                   (-70000.0, -60000.0), (3.0e38, 3.4e38)])
def test_round_f16_bit_exact(cuda, lo, hi):
    from vllm_webgpu_amd import ops

    ref = O.check_round_f16(lo, hi)
    h, c = ops.math_selftest(3, O.key(lo), O.key(hi))
    assert c == ref["count"]
    assert h == ref["hash"]


def _f16(w):
    """The workload with its logits rounded to float16 (kept as float16)."""
    w.logits = w.logits_f32().astype(np.float16)
    w.dtype = "f16"
    return w


def test_headline_shape_f16(cuda):
    """C3 (penalties, T=0.7, top-k 50, top-p 0.9) at its full shape with f16 logits."""
    w = _f16(W.config(3))
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), "C3 f16")


@pytest.mark.parametrize("cfg,scale", [(2, 1.0), (4, 0.25), (5, 0.25), (1, 1.0)])
def test_configs_f16(cuda, cfg, scale):
    w = _f16(W.config(cfg, scale))
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), f"C{cfg} f16")
    if cfg == 5:
        assert int(((g["flags"] & STREAM) != 0).sum()) >= 0.8 * w.shape[0]


def test_top_p_and_logprobs_f16(cuda):
    rng = np.random.default_rng(30)
    x = (rng.normal(0, 3, (16, 70000)) + W._zipf_bias(rng, 70000, 1.2)[None, :]).astype(np.float16)
    T = np.array([1.0, 0.7, 1.3, 0.0] * 4, np.float32)
    w = _wl("topp f16", x, T, p=0.9, seed=30, dtype="f16", L=5)
    assert_same(gpu_run(w, cuda), oracle_run(w), w.name)


def test_wide_rows_f16(cuda):
    rng = np.random.default_rng(31)
    x = rng.normal(0, 1.5, (8, 100000)).astype(np.float16)
    w = _wl("wide f16", x, 1.4, p=0.995, seed=31, dtype="f16")
    assert_same(gpu_run(w, cuda), oracle_run(w), w.name)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_softcap_f16_store(cuda, dtype):
    """Greedy rows whose capped maxima tie only after the f16 rounding (the lowest index wins),
    and sampled rows (single pass, multi-pass, top-p stream is not used with the cap)."""
    rng = np.random.default_rng(32)
    B, V = 16, 50000
    x = (rng.standard_normal((B, V)) * 25.0).astype(np.float32)
    x[0, [100, 2000, 3000]] = [70.0, 70.01, 70.02]
    x[1, [7, 8]] = [55.0, 55.004]
    x[2, [40000, 10]] = [66.0, 66.003]
    if dtype == "f16":
        x = x.astype(np.float16)
    T = np.where(np.arange(B) < 4, 0.0, 0.8).astype(np.float32)
    k = np.array([0] * 4 + [50, 1, 20, 100, 256, 0, 0, 50, 5, 64, 65, 30], np.int32)
    w = _wl(f"cap f16 store {dtype}", x, T, k=k, p=0.9, seed=32, dtype=dtype)
    capped = O.softcap_row(w.logits_f32()[0], 30.0, round_f16=True)
    assert capped[100] == capped[2000] == capped[3000]
    g = gpu_run(w, cuda, softcap=30.0, softcap_f16=True)
    assert_same(g, oracle_run(w, softcap=30.0, softcap_f16=True), w.name)
    g2 = gpu_run(w, cuda, num_logprobs=4, softcap=30.0, softcap_f16=True)
    assert_same(g2, oracle_run(w, num_logprobs=4, softcap=30.0, softcap_f16=True), w.name + " L=4")


def test_ops_f16(cuda):
    """argmax, top-k and softmax take f16 rows as they are."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(33)
    x = (np.round(rng.normal(size=(8, 30011)) * 8) / 8).astype(np.float16)  # ties
    x[1, [5, 900]] = np.float16(60000.0)
    xf = x.astype(np.float32)
    t = torch.from_numpy(x).to(cuda)
    assert np.array_equal(ops.argmax(t).cpu().numpy(), O.argmax(xf))
    for k in (1, 50, 256):
        vals, ids = ops.topk(t, k)
        rv, ri = O.topk(xf, k)
        assert np.array_equal(ids.cpu().numpy(), ri)
        assert np.array_equal(vals.cpu().numpy(), rv)
    p, rm, _ = ops.softmax(t, torch.full((8,), 0.9))
    for b in range(8):
        rp, rrm, _ = O.softmax(xf[b:b + 1], 0.9)
        np.testing.assert_allclose(p.cpu().numpy()[b], rp[0], rtol=1e-5, atol=1e-12)
        assert rm.cpu().numpy()[b] == rrm[0]


@pytest.mark.parametrize("cap", [None, 30.0])
def test_sampler_forward_f16_logits_without_cast(cuda, cap):
    """The v1 Sampler takes a float16 logits tensor as it is (and with the cap stored in f16)
    and matches the oracle on the widened logits and the same uniforms."""
    import torch

    from tests.test_gpu_v1 import _gens, _metadata
    from vllm_webgpu_amd.v1.sample.sampler import Sampler, draw_seeds

    w = _f16(W.config(3, 0.05))
    B, V = w.shape
    logits = torch.from_numpy(w.logits).to(cuda)
    assert logits.dtype == torch.float16
    out = Sampler(logit_softcap=cap, logit_softcap_f16=cap is not None)(
        logits, _metadata(w, cuda, _gens(B, cuda, 7100), 3))
    u = O.philox_uniforms(draw_seeds(B, _gens(B, cuda, 7100), cuda).cpu().numpy(), V)
    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                        w.frequency)
    ref = O.sample(w.logits_f32(), prm, u, output_ids=w.output_ids, num_logprobs=3, softcap=cap,
                   softcap_f16=cap is not None)
    assert np.array_equal(out.sampled_token_ids.cpu().numpy()[:, 0], ref["token"])
    lp = out.logprobs_tensors
    np.testing.assert_array_equal(lp.logprob_token_ids.cpu().numpy(), ref["lp_ids"])
    np.testing.assert_array_equal(lp.selected_token_ranks.cpu().numpy(), ref["ranks"])
    np.testing.assert_allclose(lp.logprobs.cpu().numpy(), ref["lp_vals"], rtol=1e-5, atol=1e-6)

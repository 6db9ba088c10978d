"""GPU parity: the HIP sampler against the CPU oracle on the same seeded inputs.

Token ids, survivor counts and result flags must be bit-exact; raw logprob values match within
rtol 1e-5.  Inputs: the five benchmark configurations at reduced size (the oracle finishes in
seconds), the crafted edge cases of tests/cases.py, and the reference's own planted known
answers (vllm_webgpu tests/test_kernels_sample.py, tests/test_kernels_attn.py)."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import all_cases
from tests.common import assert_same, gpu_run, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu


def test_library_loads_and_abi(cuda):
    from vllm_webgpu_amd import _lib

    assert _lib.lib().vws_abi_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("fn,lo,hi", [
    (0, -80.0, -40.0), (0, -1.0, -0.25), (0, -2.0 ** -10, -2.0 ** -14), (0, -0.5, 0.5),
    (1, 1e-45, 1e-38), (1, 0.25, 1.0), (1, 1.0, 4.0),
])
def test_math_bit_exact(cuda, fn, lo, hi):
    """exp_det / log_det on the GPU give the oracle's bits on every fp32 of the range."""
    from vllm_webgpu_amd import ops

    ref = O.check_exp(lo, hi) if fn == 0 else O.check_log(lo, hi)
    h, c = ops.math_selftest(fn, O.key(lo), O.key(hi))
    assert c == ref["count"]
    assert h == ref["hash"]


def test_argmax_planted_and_ties(cuda):
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(5)
    x = rng.normal(size=(16, 40000)).astype(np.float32)
    x[0, 77] = 100.0
    x[1, [5, 900, 39999]] = 50.0       # ties: lowest index wins
    x[2, :] = 1.0                      # all equal -> 0
    x[3, 17] = np.nan                  # NaN never selected
    x[4, :] = np.nan
    x[4, 123] = -1.0
    got = ops.argmax(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert np.array_equal(got, O.argmax(x))
    assert got[0] == 77 and got[1] == 5 and got[2] == 0 and got[4] == 123


def test_argmax_bf16_unaligned(cuda):
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(6)
    x = rng.normal(size=(7, 50257)).astype(np.float32)
    t = torch.from_numpy(x).to(cuda).to(torch.bfloat16)
    ref = O.argmax(t.float().cpu().numpy())
    assert np.array_equal(ops.argmax(t).cpu().numpy(), ref)


def test_topk_planted(cuda):
    """vllm_webgpu tests/test_kernels_sample.py:51-101: values [10,9,8,7,6] at [77,3,100,50,22]."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(7)
    x = rng.normal(size=(1, 128)).astype(np.float16).astype(np.float32)
    for i, v in zip([77, 3, 100, 50, 22], [10.0, 9.0, 8.0, 7.0, 6.0]):
        x[0, i] = v
    vals, ids = ops.topk(torch.from_numpy(x).to(cuda), 5)
    assert ids.cpu().numpy().tolist() == [[77, 3, 100, 50, 22]]
    assert np.all(np.diff(vals.cpu().numpy()[0]) <= 0)


@pytest.mark.parametrize("k", [1, 7, 50, 256])
def test_topk_random(cuda, k):
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(8 + k)
    x = np.round(rng.normal(size=(12, 30011)) * 8).astype(np.float32) / 8  # ties
    vals, ids = ops.topk(torch.from_numpy(x).to(cuda), k)
    rv, ri = O.topk(x, k)
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.array_equal(vals.cpu().numpy(), rv)


def test_softmax(cuda):
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(9)
    x = (rng.normal(size=(6, 32000)) * 3).astype(np.float32)
    T = np.array([1.0, 0.5, 2.0, 1.0, 0.8, 1.3], np.float32)
    p, rm, ls = ops.softmax(torch.from_numpy(x).to(cuda), torch.from_numpy(T))
    p = p.cpu().numpy()
    for b in range(6):
        rp, rrm, rls = O.softmax(x[b:b + 1], float(T[b]))
        np.testing.assert_allclose(p[b], rp[0], rtol=1e-5, atol=1e-12)
        assert rm.cpu().numpy()[b] == rrm[0]
    np.testing.assert_allclose(p.sum(1), 1.0, rtol=1e-5)
    # translation invariance (vllm_webgpu tests/test_kernels_attn.py:228-273)
    for shift in (5.0, -5.0, 100.0):
        q, _, _ = ops.softmax(torch.from_numpy(x + np.float32(shift)).to(cuda), torch.from_numpy(T))
        np.testing.assert_allclose(q.cpu().numpy(), p, rtol=2e-4, atol=1e-9)


def test_softmax_long_rows(cuda):
    """Rows longer than 32 values per thread (the two-read path: an online max and normaliser,
    then the write), with -inf and NaN elements (exp_det is 0 for NaN: their probability is 0),
    a row of one finite value, and a row in ascending order (every thread's running maximum
    rises at each of its values)."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(19)
    B, V = 5, 150001
    x = (rng.normal(size=(B, V)) * 3).astype(np.float32)
    x[1, ::7] = -np.inf
    x[2, 1234] = np.nan
    x[3, :] = -np.inf
    x[3, 77] = 2.5
    x[4] = np.sort(x[4])
    T = np.array([1.0, 0.7, 1.5, 1.0, 0.9], np.float32)
    p, rm, ls = ops.softmax(torch.from_numpy(x).to(cuda), torch.from_numpy(T))
    p, rm, ls = p.cpu().numpy(), rm.cpu().numpy(), ls.cpu().numpy()
    for b in range(B):
        rp, rrm, rls = O.softmax(x[b:b + 1], float(T[b]))
        np.testing.assert_allclose(p[b], rp[0], rtol=1e-5, atol=1e-12, equal_nan=True)
        assert rm[b] == rrm[0]
        np.testing.assert_allclose(ls[b], rls[0], rtol=1e-6)
    assert p[3, 77] == 1.0 and not p[3, :77].any()


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("scale", [0.05, 0.25])
def test_config_scaled(cuda, cfg, scale):
    w = W.config(cfg, scale=scale)
    ref = oracle_run(w)
    got = gpu_run(w, cuda)
    assert_same(got, ref, f"C{cfg}@{scale}")


@pytest.mark.parametrize("case", all_cases(), ids=lambda w: w.name)
def test_edge_cases(cuda, case):
    ref = oracle_run(case)
    got = gpu_run(case, cuda)
    assert_same(got, ref, case.name)


def test_repeat_calls_stable(cuda):
    """Workspace stays clean between calls: three calls give identical results."""
    w = W.config(3, scale=0.1)
    first = gpu_run(w, cuda)
    for _ in range(2):
        again = gpu_run(w, cuda)
        assert np.array_equal(again["token"], first["token"])
        assert np.array_equal(again["n_kept"], first["n_kept"])


def test_workspace_clean_after_general_path(cuda):
    """The multi-pass path keeps its history hash in the shared workspace; it must leave zeros
    behind, since the top-k operation's part counters overlap that region."""
    import torch

    from tests.cases import _wl
    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(21)
    B, V, H = 8, 20000, 400
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    w = _wl("general_with_history", x, 0.9, k=0, p=0.9, rep=1.2, pres=0.3, freq=0.1, hist=hist, seed=9)
    assert_same(gpu_run(w, cuda), oracle_run(w), w.name)
    xt = np.round(rng.normal(size=(12, 30011)) * 8).astype(np.float32) / 8
    for k in (1, 50):
        vals, ids = ops.topk(torch.from_numpy(xt).to(cuda), k)
        rv, ri = O.topk(xt, k)
        assert np.array_equal(ids.cpu().numpy(), ri)
        assert np.array_equal(vals.cpu().numpy(), rv)

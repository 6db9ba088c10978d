"""GPU parity at the benchmark configurations' real sizes.

Every configuration runs at its stated B x V (``workloads.config(i)``, scale 1.0) through
``vws_sample`` and through the CPU oracle on the same seeded inputs.  Token ids, the low byte of
the result flags (near-tie, degenerate, greedy), survivor counts, logprob ids and ranks must be
identical; logprob values agree within rtol 1e-5 (fp32 logits, and bf16 logits, which both
sides widen exactly).  At these sizes the single pass streams many iterations per row (C3: four
per wave), raises its threshold mid-stream and compacts candidate buffers; the multi-pass path
serves C4's rows without top-k and every C5 row.

C1 (greedy argmax + temperature-1 softmax over [1, 32000]) checks ``vws_sample`` in greedy mode
and ``vws_softmax`` (probabilities within rtol 1e-5 of the oracle's, row max bit-exact).
"""
import functools

import numpy as np
import pytest

from oracle import sampler as O
from tests.common import assert_same, gpu_run, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=2)
def _config(i):
    return W.config(i)


def _summary(res):
    fl = res["flags"] & 0xFF
    return (f"kept mean {res['n_kept'].mean():.1f}, top-p near ties {int(((fl & 1) != 0).sum())}, "
            f"race near ties {int(((fl & 2) != 0).sum())}, greedy {int(((fl & 8) != 0).sum())}")


def test_c1_greedy_and_softmax_full(cuda):
    import torch

    from vllm_webgpu_amd import ops

    w = _config(1)
    assert w.shape == (1, 32000)
    x = torch.from_numpy(w.logits).to(cuda)
    ref = oracle_run(w)
    got = gpu_run(w, cuda)
    assert_same(got, ref, "C1")
    assert got["token"][0] == int(np.argmax(w.logits[0]))
    p, rm, ls = ops.softmax(x, torch.ones(1))
    torch.cuda.synchronize()
    rp, rrm, rls = O.softmax(w.logits, 1.0)
    np.testing.assert_allclose(p.cpu().numpy(), rp, rtol=1e-5, atol=1e-12)
    assert rm.cpu().numpy()[0] == rrm[0]
    np.testing.assert_allclose(ls.cpu().numpy()[0], rls[0], rtol=1e-6)


@pytest.mark.parametrize("cfg", [2, 3, 4, 5])
def test_config_full(cuda, cfg):
    w = _config(cfg)
    print(f"C{cfg} {w.shape} {w.dtype}", flush=True)
    ref = oracle_run(w)
    got = gpu_run(w, cuda)
    print(f"C{cfg}: oracle {_summary(ref)}; gpu {_summary(got)}", flush=True)
    assert_same(got, ref, f"C{cfg} full size")


def test_c4_full_with_logprobs(cuda):
    """bf16 logits with raw logprobs: every row goes through the logprob passes."""
    w = _config(4)
    ref = oracle_run(w, num_logprobs=20)
    got = gpu_run(w, cuda, num_logprobs=20)
    assert_same(got, ref, "C4 full size + 20 logprobs")


def test_c3_full_repeated_rotated(cuda):
    """The benchmark's rotation (rows rolled by one) gives the rolled results."""
    w = _config(3)
    ref = oracle_run(w)
    rolled = W.Workload(w.name, np.roll(w.logits, 1, axis=0), w.dtype, w.temperature, w.top_k,
                        w.top_p, w.min_p, w.repetition, w.presence, w.frequency,
                        np.roll(w.output_ids, 1, axis=0), np.roll(w.uniforms, 1, axis=0))
    got = gpu_run(rolled, cuda)
    assert np.array_equal(got["token"], np.roll(ref["token"], 1))
    assert np.array_equal(got["n_kept"], np.roll(ref["n_kept"], 1))

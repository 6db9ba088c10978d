"""The oracle against the torch-CPU statement of the vLLM-v1 sampler (``oracle/vllm_torch.py``),
which is also bench.py's CPU baseline: the two are written independently (exact integer masses
and order keys vs. float softmax, sort and cumsum), so agreement on every row that is not a
near tie pins both to the same semantics."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sampler as O
from oracle import vllm_torch as VT
from tests.common import oracle_run
from vllm_webgpu_amd import workloads


def _torch_run(w, compute_dtype):
    x = torch.from_numpy(w.logits_f32())
    hist = torch.from_numpy(w.output_ids) if w.output_ids is not None else None
    u = torch.from_numpy(w.uniforms) if w.uniforms is not None else torch.full(w.shape, 0.5)
    return VT.sample(x, torch.from_numpy(w.temperature), torch.from_numpy(w.top_k),
                     torch.from_numpy(w.top_p), torch.from_numpy(w.min_p),
                     torch.from_numpy(w.repetition), torch.from_numpy(w.presence),
                     torch.from_numpy(w.frequency), u, output_ids=hist,
                     num_logprobs=w.num_logprobs, compute_dtype=compute_dtype)


@pytest.mark.parametrize("cfg,scale", [(2, 0.25), (3, 0.1), (4, 0.05), (5, 0.03)])
def test_tokens_agree_off_near_ties(cfg, scale):
    w = workloads.config(cfg, scale)
    ref = oracle_run(w)
    got = _torch_run(w, torch.float64)
    near = (ref["flags"] & (O.FLAG_TOPP_NEAR_TIE | O.FLAG_RACE_NEAR_TIE)) != 0
    tok = got["token"].numpy()
    bad = np.nonzero((tok != ref["token"]) & ~near)[0]
    assert bad.size == 0, (bad[:8], tok[bad[:8]], ref["token"][bad[:8]])
    nk = got["n_kept"].numpy()
    badk = np.nonzero((nk != ref["n_kept"]) & ~near)[0]
    assert badk.size == 0, (badk[:8], nk[badk[:8]], ref["n_kept"][badk[:8]])
    assert near.mean() < 0.05
    if w.num_logprobs is not None:
        ok = ~near
        assert np.array_equal(got["ranks"].numpy()[ok], ref["ranks"][ok])
        np.testing.assert_allclose(got["lp_vals"].numpy()[ok], ref["lp_vals"][ok], rtol=1e-5,
                                   atol=1e-5)


def test_float32_baseline_agrees_on_almost_every_row():
    # the fp32 form bench.py times differs only where fp32 rounding moves a boundary
    w = workloads.config(2, 0.25)
    ref = oracle_run(w)
    got = _torch_run(w, torch.float32)
    assert (got["token"].numpy() == ref["token"]).mean() >= 0.95

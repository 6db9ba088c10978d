"""Shared helpers for the parity tests: run a workload through the oracle and through the GPU
library on the same inputs and compare (token ids bit-exact, logprob values by tolerance)."""
from __future__ import annotations

import numpy as np

from oracle import sampler as O

# Result flags compared between the GPU and the oracle (diagnostic bits above 0xFF excluded).
FLAG_MASK = 0xFF
# Raw logprobs are floating point: tolerance of the north star for fp32 logits.
LP_RTOL = 1e-5
LP_ATOL = 1e-6


def oracle_run(w, num_logprobs=None, softcap=None, softcap_f16=False):
    B = w.shape[0]
    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                        w.frequency)
    return O.sample(w.logits_f32(), prm, w.uniforms, output_ids=w.output_ids,
                    num_logprobs=w.num_logprobs if num_logprobs is None else num_logprobs,
                    softcap=softcap, softcap_f16=softcap_f16)


def gpu_run(w, device, num_logprobs=None, softcap=None, softcap_f16=False):
    import torch

    from vllm_webgpu_amd import ops

    if w.dtype == "bf16":
        logits = torch.from_numpy(w.logits.view(np.int16)).to(device).view(torch.bfloat16)
    else:  # float32 or float16, sampled as they are
        logits = torch.from_numpy(w.logits).to(device)
    greedy_all = bool(np.all(~(w.temperature >= np.float32(1e-5))))
    T = torch.from_numpy(w.temperature)
    U = torch.from_numpy(w.uniforms).to(device) if w.uniforms is not None else None
    if U is None and not greedy_all:
        U = torch.full(w.shape, 0.5, dtype=torch.float32, device=device)
    hist = torch.from_numpy(w.output_ids) if w.output_ids is not None else None
    L = w.num_logprobs if num_logprobs is None else num_logprobs
    res = ops.sample(logits, temperature=None if greedy_all else T, top_k=torch.from_numpy(w.top_k),
                     top_p=torch.from_numpy(w.top_p), min_p=torch.from_numpy(w.min_p),
                     repetition_penalty=torch.from_numpy(w.repetition),
                     presence_penalty=torch.from_numpy(w.presence),
                     frequency_penalty=torch.from_numpy(w.frequency), output_ids=hist,
                     uniforms=U, num_logprobs=L, logit_softcap=softcap,
                     logit_softcap_f16=softcap_f16)
    torch.cuda.synchronize()
    out = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
               n_kept=res.num_kept.cpu().numpy())
    if L is not None:
        out.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                   ranks=res.logprob_ranks.cpu().numpy())
    return out


def assert_same(gpu, ref, label=""):
    bad = np.nonzero(gpu["token"] != ref["token"])[0]
    assert bad.size == 0, (f"{label}: token mismatch in {bad.size} rows, first {bad[:8]}: "
                           f"gpu {gpu['token'][bad[:8]]} oracle {ref['token'][bad[:8]]} "
                           f"flags {gpu['flags'][bad[:8]]}")
    fl = (gpu["flags"] & FLAG_MASK) != (ref["flags"] & FLAG_MASK)
    assert not fl.any(), (f"{label}: flag mismatch rows {np.nonzero(fl)[0][:8]}: "
                          f"gpu {gpu['flags'][fl][:8]} oracle {ref['flags'][fl][:8]}")
    nk = gpu["n_kept"] != ref["n_kept"]
    assert not nk.any(), (f"{label}: n_kept mismatch rows {np.nonzero(nk)[0][:8]}: "
                          f"gpu {gpu['n_kept'][nk][:8]} oracle {ref['n_kept'][nk][:8]}")
    if "lp_ids" in ref:
        bad = np.nonzero((gpu["lp_ids"] != ref["lp_ids"]).any(axis=1))[0]
        assert bad.size == 0, (f"{label}: logprob ids differ in rows {bad[:8]} (flags "
                               f"{gpu['flags'][bad[:8]]}): gpu {gpu['lp_ids'][bad[:2]].tolist()} "
                               f"oracle {ref['lp_ids'][bad[:2]].tolist()}")
        bad = np.nonzero(gpu["ranks"] != ref["ranks"])[0]
        assert bad.size == 0, (f"{label}: ranks differ in rows {bad[:8]}: gpu {gpu['ranks'][bad[:8]]} "
                               f"oracle {ref['ranks'][bad[:8]]}")
        np.testing.assert_allclose(gpu["lp_vals"], ref["lp_vals"], rtol=LP_RTOL, atol=LP_ATOL,
                                   err_msg=f"{label}: logprob values")

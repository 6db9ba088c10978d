"""vws_sample_noalloc (static device scratch, no allocation) against vws_sample (caller
workspace) through the C ABI: identical outputs on two calls in a row, the second with a smaller
batch, vocabulary and history, and both identical to the CPU oracle.

Half the rows of each batch have top-k off, so the multi-pass path serves them and keeps their
history hash in the scratch; the other rows take the single pass.  The two calls share the one
static scratch (the second call reuses what the first left behind), and the same launches with
a caller workspace give the reference outputs.
"""
import ctypes

import numpy as np
import pytest

from oracle import sampler as O

pytestmark = pytest.mark.gpu


def _inputs(seed, B, V, H):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    hist = rng.integers(0, V + 40, (B, H)).astype(np.int32)        # ids >= V are padding
    T = rng.uniform(0.5, 1.2, B).astype(np.float32)
    T[::5] = 0.0                                                    # greedy rows
    k = np.where(np.arange(B) % 2 == 0, 0, 40).astype(np.int32)     # even rows: top-k off
    p = rng.uniform(0.6, 0.95, B).astype(np.float32)
    u = (rng.integers(1, 2 ** 24, (B, V)).astype(np.float32) * np.float32(2.0 ** -24))
    return dict(x=x, hist=hist, T=T, k=k, p=p, u=u,
                rep=np.full(B, 1.2, np.float32), pres=np.full(B, 0.4, np.float32),
                freq=np.full(B, 0.1, np.float32))


def _run(entry, d, dev, with_ws):
    import torch

    from vllm_webgpu_amd import _lib, ops

    L = _lib.lib()
    B, V = d["x"].shape
    t = {k: torch.from_numpy(v).to(dev) for k, v in d.items()}
    out = torch.full((B,), -7, dtype=torch.int32, device=dev)
    flags = torch.full((B,), -7, dtype=torch.int32, device=dev)
    kept = torch.full((B,), -7, dtype=torch.int32, device=dev)
    a = _lib.SampleArgs()
    a.struct_size = ctypes.sizeof(_lib.SampleArgs)
    a.batch, a.vocab, a.dtype = B, V, _lib.DTYPE_F32
    a.logits, a.logits_row_stride = t["x"].data_ptr(), V
    a.temperature, a.top_k, a.top_p = t["T"].data_ptr(), t["k"].data_ptr(), t["p"].data_ptr()
    a.repetition_penalty, a.presence_penalty = t["rep"].data_ptr(), t["pres"].data_ptr()
    a.frequency_penalty = t["freq"].data_ptr()
    a.output_ids, a.output_row_stride, a.output_width = t["hist"].data_ptr(), d["hist"].shape[1], d["hist"].shape[1]
    a.uniforms, a.uniforms_row_stride = t["u"].data_ptr(), V
    a.sampled, a.row_flags, a.num_kept = out.data_ptr(), flags.data_ptr(), kept.data_ptr()
    a.num_logprobs = -1
    ws = None
    if with_ws:
        ws = ops.workspace(L.vws_sample_workspace_size(B, V, d["hist"].shape[1]), dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.stream = torch.cuda.current_stream().cuda_stream
    _lib.check(entry(ctypes.byref(a)))
    torch.cuda.synchronize()
    return dict(token=out.cpu().numpy(), flags=flags.cpu().numpy().view(np.uint32),
                n_kept=kept.cpu().numpy())


def _oracle(d):
    B = d["x"].shape[0]
    prm = O.make_params(B, d["T"], d["k"], d["p"], 0.0, d["rep"], d["pres"], d["freq"])
    return O.sample(d["x"], prm, d["u"], output_ids=d["hist"])


def test_noalloc_matches_workspace_entry_twice(cuda):
    from vllm_webgpu_amd import _lib

    L = _lib.lib()
    for call, (seed, B, V, H) in enumerate([(1, 64, 32000, 512), (2, 16, 20000, 100)]):
        print(f"no-alloc call {call}: B={B} V={V} H={H}", flush=True)
        d = _inputs(seed, B, V, H)
        need = L.vws_sample_workspace_size(B, V, H)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
        ref = _run(L.vws_sample, d, cuda, True)
        got = _run(L.vws_sample_noalloc, d, cuda, False)
        for key in ("token", "n_kept"):
            assert np.array_equal(got[key], ref[key]), f"call {call}: {key}"
        assert np.array_equal(got["flags"], ref["flags"]), f"call {call}: flags"
        orc = _oracle(d)
        assert np.array_equal(got["token"], orc["token"]), f"call {call}: oracle tokens"
        assert np.array_equal(got["n_kept"], orc["n_kept"]), f"call {call}: oracle n_kept"
        assert np.array_equal(got["flags"] & 0xFF, orc["flags"] & 0xFF), f"call {call}: oracle flags"
        assert (got["flags"] & _lib.FLAG_GENERAL_PATH).any(), "no row used the scratch"


def test_noalloc_rejects_batches_beyond_the_scratch(cuda):
    from vllm_webgpu_amd import _lib

    L = _lib.lib()
    a = _lib.SampleArgs()
    a.struct_size = ctypes.sizeof(_lib.SampleArgs)
    a.batch, a.vocab, a.dtype = 4096, 1000, _lib.DTYPE_F32
    a.logits, a.logits_row_stride, a.sampled = 0x10000, 1000, 0x10000
    a.output_ids, a.output_row_stride, a.output_width = 0x10000, 2048, 2048
    a.num_logprobs = -1
    assert L.vws_sample_workspace_size(4096, 1000, 2048) > _lib.NOALLOC_SCRATCH_BYTES
    assert L.vws_sample_noalloc(ctypes.byref(a)) == _lib.ERR_LIMIT
    assert "static scratch" in _lib.last_error()


@pytest.mark.parametrize("seed", range(16))
def test_noalloc_matches_the_workspace_entry_on_random_launches(cuda, seed):
    """Random mixed launches (every sampling option; see tests/test_gpu_random_mix.py) prepared
    once, run through vws_sample and then through vws_sample_noalloc with the same arguments:
    tokens, flags, survivor counts, logprob ids and ranks identical, logprob values within
    1e-6 (the device's double sums may finish in another order)."""
    import torch

    from tests.cases import _u
    from tests.test_gpu_random_mix import _launch, _words
    from vllm_webgpu_amd import _lib, ops

    L = _lib.lib()
    rng = np.random.default_rng(31000 + seed)
    c = _launch(rng, ["f32", "bf16", "f16"][seed % 3], big=seed % 5 == 4)
    B, V = c["B"], c["V"]
    u = _u(rng, (B, V))
    bits = None if c["allowed"] is None else _words(c["allowed"])
    if c["dt"] == "bf16":
        x = torch.from_numpy(c["raw"].view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        x = torch.from_numpy(c["raw"]).to(cuda)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    greedy_all = bool(np.all(~(c["T"] >= np.float32(1e-5))))
    prep = ops.prepare_sample(
        x, temperature=None if greedy_all else torch.from_numpy(c["T"]),
        top_k=torch.from_numpy(c["k"]), top_p=torch.from_numpy(c["p"]),
        min_p=torch.from_numpy(c["mp"]), repetition_penalty=torch.from_numpy(c["rep"]),
        presence_penalty=torch.from_numpy(c["pres"]), frequency_penalty=torch.from_numpy(c["freq"]),
        prompt_ids=t(c["prompt"]), output_ids=t(c["output"]), uniforms=t(u),
        num_logprobs=c["L"], allowed_mask=None if bits is None else t(bits.view(np.int32)),
        adjust_ids=t(c["aid"]), adjust_vals=t(c["aval"]), adjust_lens=t(c["alen"]),
        logit_softcap=c["cap"], logit_softcap_f16=c["cap16"])
    if L.vws_sample_workspace_size(B, V, prep.args.prompt_width + prep.args.output_width) > _lib.NOALLOC_SCRATCH_BYTES:
        pytest.skip("beyond the static scratch")
    res = prep.launch()
    outs = [res.sampled, res.flags, res.num_kept]
    if c["L"] is not None:
        outs += [res.logprob_ids, res.logprob_ranks, res.logprob_vals]
    torch.cuda.synchronize()
    ref = [o.cpu().numpy().copy() for o in outs]
    for o in outs:
        o.fill_(-7)
    prep.args.stream = ops._stream_ptr()
    _lib.check(L.vws_sample_noalloc(ctypes.byref(prep.args)))
    torch.cuda.synchronize()
    got = [o.cpu().numpy() for o in outs]
    label = f"seed {seed}: {c['dt']} B={B} V={V} L={c['L']}"
    for g, r in zip(got[:-1] if c["L"] is not None else got, ref):
        assert np.array_equal(g, r), label
    if c["L"] is not None:
        np.testing.assert_allclose(got[-1], ref[-1], rtol=1e-6, atol=0, equal_nan=True, err_msg=label)

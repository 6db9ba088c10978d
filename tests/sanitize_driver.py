"""Runs the host-side code of the library and the CPU oracle under AddressSanitizer and
UndefinedBehaviorSanitizer (started by tests/test_sanitized_host.py in a child process with the
sanitizer runtime preloaded; any report aborts that process).

It loads the host-only sanitized build of the C ABI (vllm_webgpu_amd/csrc/_san/_vws_host.so: no
device code, so only calls that return before a launch are made) and the sanitized oracle
(oracle/_san/liboracle.so), without torch.  Exercised: every argument check of vws_sample and
the operations, workspace sizes over a grid of shapes, the token-state and test-hook entry
points, the profiling entry points' failure paths, and the oracle on the crafted edge cases
(ties, -inf, NaN, penalties, processors, logprobs, soft cap, generated uniforms)."""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from vllm_webgpu_amd import _lib  # noqa: E402  (ctypes mirror only; torch is not imported)

FAKE = 0x10000000


def capi():
    L = ctypes.CDLL(os.path.join(ROOT, "vllm_webgpu_amd", "csrc", "_san", "_vws_host.so"))
    _lib._declare(L)
    assert L.vws_abi_version() == _lib.ABI_VERSION

    def args(**over):
        a = _lib.SampleArgs()
        a.struct_size = ctypes.sizeof(_lib.SampleArgs)
        a.batch, a.vocab, a.dtype = 4, 1000, _lib.DTYPE_F32
        a.logits, a.logits_row_stride = FAKE, 1000
        a.temperature, a.uniforms, a.uniforms_row_stride = FAKE, FAKE, 1000
        a.sampled, a.num_logprobs = FAKE, -1
        a.workspace, a.workspace_bytes = 0x100000, L.vws_sample_workspace_size(4, 1000, 0)
        for k, v in over.items():
            setattr(a, k, v)
        return a

    hist = dict(output_ids=FAKE, output_width=8, output_row_stride=8)
    bad = [dict(logits=None), dict(batch=0), dict(batch=-5), dict(vocab=0), dict(vocab=(1 << 19) + 1),
           dict(dtype=7), dict(logits_row_stride=999), dict(sampled=None), dict(uniforms=None),
           dict(uniforms_row_stride=10), dict(num_logprobs=65), dict(num_logprobs=-2),
           dict(num_logprobs=5), dict(prompt_ids=FAKE, prompt_width=-1),
           dict(prompt_ids=FAKE, prompt_width=1 << 25, prompt_row_stride=1 << 25),
           dict(output_ids=FAKE, output_width=8, output_row_stride=4),
           dict(hist, workspace=None), dict(hist, workspace_bytes=256),
           dict(hist, workspace=0x100010, workspace_bytes=1 << 20), dict(struct_size=8),
           dict(struct_size=0xFFFFFFFF), dict(adjust_ids=FAKE, adjust_width=4, adjust_row_stride=4),
           dict(adjust_ids=FAKE, adjust_vals=FAKE, adjust_width=8, adjust_row_stride=4),
           dict(allowed_mask=FAKE, allowed_row_stride=31), dict(logit_softcap=-1.0),
           dict(logit_softcap=float("nan")), dict(logit_softcap=float("inf")),
           dict(token_state=FAKE, token_state_row_stride=999),
           dict(hist, token_state=FAKE, token_state_row_stride=1000),
           dict(token_state=FAKE, token_state_row_stride=1000, token_state_bits=FAKE,
                token_state_bits_stride=31),
           dict(token_state_bits=FAKE, token_state_bits_stride=32)]
    for over in bad:
        a = args(**over)
        st = L.vws_validate_sample_args(ctypes.byref(a))
        assert st != 0, over
        assert L.vws_last_error(), over
        assert L.vws_sample(ctypes.byref(a)) == st          # rejected before any launch
        assert L.vws_sample_noalloc(ctypes.byref(a)) != 0
    assert L.vws_validate_sample_args(None) == _lib.ERR_INVALID_ARGUMENT
    for over in (dict(), dict(workspace=None, workspace_bytes=0),
                 dict(token_state=FAKE, token_state_row_stride=1000, workspace=None),
                 dict(token_state=FAKE, token_state_row_stride=1000, token_state_bits=FAKE,
                      token_state_bits_stride=32, workspace=None),
                 dict(hist, workspace_bytes=L.vws_sample_workspace_size(4, 1000, 8)),
                 dict(temperature=None, uniforms=None), dict(uniforms=None, rng_seeds=FAKE)):
        assert L.vws_validate_sample_args(ctypes.byref(args(**over))) == 0, over
    # workspace sizes over a grid (including the largest batch and history the layout allows)
    for B in (1, 7, 256, 4096, (1 << 20) - 1):
        for V in (1, 64, 32000, 1 << 19):
            for H in (0, 1, 512, 1 << 16):
                assert L.vws_sample_workspace_size(B, V, H) > 0
                assert L.vws_topk_workspace_size(B, V, 50) > 0
    assert L.vws_sample_workspace_size(0, 1, 0) == 0 and L.vws_sample_workspace_size(1, 1, -1) == 0
    # the operations' argument checks (each returns before its launch)
    assert L.vws_argmax(None, 0, 4, 1000, 1000, FAKE, None) != 0
    assert L.vws_argmax(FAKE, 0, 4, 1000, 1000, None, None) != 0
    assert L.vws_topk(FAKE, 0, 4, 1000, 1000, 0, FAKE, FAKE, FAKE, 1 << 30, None) != 0
    assert L.vws_topk(FAKE, 0, 4, 1000, 1000, 300, FAKE, FAKE, FAKE, 1 << 30, None) != 0
    assert L.vws_topk(FAKE, 0, 4, 1000, 1000, 10, FAKE, FAKE, None, 0, None) != 0
    assert L.vws_softmax(FAKE, 5, 4, 1000, 1000, None, FAKE, None, None, None) != 0
    assert L.vws_softmax(FAKE, 0, 4, 1000, 1000, None, None, None, None, None) != 0
    assert L.vws_apply_penalties(FAKE, 4, 1000, 1000, None, None, None, None, 0, 0, None, None,
                                 0, 0, None, None, 0, None) == 0
    assert L.vws_apply_penalties(FAKE, 4, 1000, 1000, None, None, None, FAKE, 8, 8, None, None,
                                 0, 0, None, None, 0, None) == _lib.ERR_WORKSPACE_TOO_SMALL
    up = L.vws_token_state_update
    assert up(None, 1000, None, 0, 1000, 1, None, 0, FAKE, 0, None) != 0
    assert up(FAKE, 999, None, 0, 1000, 1, None, 0, FAKE, 0, None) != 0
    assert up(FAKE, 1000, FAKE, 31, 1000, 1, None, 0, FAKE, 0, None) != 0
    assert up(FAKE, 1000, None, 0, 1000, 1, None, 0, FAKE, 5, None) != 0
    assert up(FAKE, 1000, None, 0, 1000, 1, None, -1, FAKE, 0, None) != 0
    assert up(FAKE, 1000, None, 0, 1000, -1, None, 0, FAKE, 0, None) != 0
    assert up(FAKE, 1000, FAKE, 32, 1000, 0, None, 0, None, 0, None) == 0
    assert L.vws_math_selftest(9, 0, 1, FAKE, None) != 0
    assert L.vws_math_selftest(0, 5, 1, FAKE, None) != 0
    prev = L.vws_set_coop_wait_polls(3)
    assert L.vws_set_coop_wait_polls(-1) == -1 and L.vws_set_coop_wait_polls(prev) == 3
    assert L.vws_profile_begin(0) != 0 and L.vws_profile_end(None, None) != 0
    L.vws_profile_begin(4)   # creates events; fails cleanly without a device
    L.vws_profile_end(None, None)
    print("C ABI host paths: ok", flush=True)


def oracle():
    from oracle import sampler as O
    from tests.cases import all_cases

    O._LIB_PATH = os.path.join(ROOT, "oracle", "_san", "liboracle.so")
    O._lib = None
    n = 0
    for w in all_cases():
        B = w.shape[0]
        prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                            w.frequency)
        O.sample(w.logits_f32(), prm, w.uniforms, output_ids=w.output_ids,
                 num_logprobs=w.num_logprobs)
        O.sample(w.logits_f32(), prm, w.uniforms, output_ids=w.output_ids, num_logprobs=3,
                 softcap=30.0, softcap_f16=True)
        n += 1
    rng = np.random.default_rng(3)
    x = rng.normal(0, 3, (6, 5000)).astype(np.float32)
    x[0, ::3] = -np.inf
    x[1, 7] = np.nan
    bits = rng.integers(0, 2 ** 32, (6, (5000 + 31) // 32), dtype=np.uint64).astype(np.uint32)
    aid = rng.integers(-3, 5003, (6, 9)).astype(np.int32)
    aval = np.where(rng.random((6, 9)) < 0.3, -np.inf, rng.normal(0, 2, (6, 9))).astype(np.float32)
    hist = rng.integers(-2, 5002, (6, 40)).astype(np.int32)
    prm = O.make_params(6, 0.8, 20, 0.9, 0.02, 1.2, 0.3, 0.1)
    u = O.philox_uniforms(np.arange(1, 7, dtype=np.uint64), 5000)
    O.sample(x, prm, u, prompt_ids=hist, output_ids=hist, allowed=bits, adjust_ids=aid,
             adjust_vals=aval, num_logprobs=8)
    O.softmax(x[2:], 0.7)
    O.topk(x[2:], 17)
    O.argmax(x)
    O.check_exp(-10.0, 10.0, 4099)
    O.check_log(1e-7, 1.0, 4099)
    print(f"oracle: {n} crafted cases and processors: ok", flush=True)


if __name__ == "__main__":
    capi()
    oracle()

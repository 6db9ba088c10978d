"""The C-ABI library on the CPU: it loads, exports every entry point that
``include/vws_sampler.h`` declares, reports its ABI version and workspace sizes, and its host
argument validation returns the documented status codes.  No compute call is made here."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from vllm_webgpu_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vws_sampler.h")


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        subprocess.run(["make", "-s", "-j4", "-C", os.path.join(ROOT, "vllm_webgpu_amd", "csrc")],
                       check=True)
    return _lib.lib()


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(vws_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.EXPORTED)


def test_exports_every_declared_symbol(L):
    for name in _declared():
        assert getattr(L, name) is not None, name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (vws_\w+)", out))
    assert set(_declared()) <= exported


def test_abi_constants_match_header(L):
    text = open(HEADER).read()

    def define(name):
        body = re.search(rf"#define {name}\s+([^/\n]+)", text).group(1).strip()
        m = re.fullmatch(r"\(\s*(\d+)\s*<<\s*(\d+)\s*\)", body)
        return (int(m.group(1)) << int(m.group(2))) if m else int(body.rstrip("u"), 0)

    assert L.vws_abi_version() == _lib.ABI_VERSION == define("VWS_ABI_VERSION")
    assert define("VWS_ERR_INVALID_ARGUMENT") == _lib.ERR_INVALID_ARGUMENT
    assert define("VWS_ERR_UNSUPPORTED_DTYPE") == _lib.ERR_UNSUPPORTED_DTYPE
    assert define("VWS_ERR_WORKSPACE_TOO_SMALL") == _lib.ERR_WORKSPACE_TOO_SMALL
    assert define("VWS_ERR_LIMIT") == _lib.ERR_LIMIT
    assert define("VWS_ERR_UNSUPPORTED") == _lib.ERR_UNSUPPORTED
    assert define("VWS_TRACE_SLOTS") == _lib.TRACE_SLOTS
    for n in ("ENTRY", "PARAMS", "FIRST", "SEED", "STREAM", "ROW", "EXIT", "WAVE_LOOP", "WAVE_PACK",
              "TP_HIST", "TP_MASS", "TP_CUT", "TP_RACE", "TP_LOGPROBS", "XCC", "ROWID"):
        assert define(f"VWS_TRACE_{n}") == getattr(_lib, f"TRACE_{n}"), n
    assert define("VWS_MAX_VOCAB") == _lib.MAX_VOCAB
    assert define("VWS_MAX_LOGPROBS") == _lib.MAX_LOGPROBS


def test_workspace_sizes(L):
    # a fixed region first (rows' shared passes, the row queue), the same for every batch
    c0 = L.vws_sample_workspace_size(256, 128256, 0)
    assert c0 > 500_000 and c0 % 256 == 0
    assert L.vws_sample_workspace_size(1, 100, 0) == c0
    assert L.vws_sample_workspace_size(4096, 262144, 0) == c0
    # then the history hash: 256 rows x 1024 slots (power of two >= 2 x 512) x 4 words
    a = L.vws_sample_workspace_size(256, 128256, 512)
    assert a == c0 + 256 * 1024 * 16
    assert L.vws_sample_workspace_size(512, 128256, 512) == c0 + 2 * 256 * 1024 * 16
    assert L.vws_sample_workspace_size(4, 100, 1) == c0 + 4 * 64 * 16  # at least 64 slots
    assert L.vws_sample_workspace_size(0, 100, 0) == 0
    assert L.vws_sample_workspace_size(4, 100, -1) == 0
    t = L.vws_topk_workspace_size(8, 1000, 50)
    assert t > 0 and t % 256 == 0


FAKE = 0x10000          # host-side stand-in addresses: validation never dereferences them


HIST = dict(output_ids=FAKE, output_width=8, output_row_stride=8)   # needs a workspace


def _args(L, **over):
    a = _lib.SampleArgs()
    a.struct_size = ctypes.sizeof(_lib.SampleArgs)
    a.batch, a.vocab, a.dtype = 4, 1000, _lib.DTYPE_F32
    a.logits, a.logits_row_stride = FAKE, 1000
    a.temperature = FAKE
    a.uniforms, a.uniforms_row_stride = FAKE, 1000
    a.sampled = FAKE
    a.num_logprobs = -1
    a.workspace = 0x100000
    a.workspace_bytes = L.vws_sample_workspace_size(4, 1000, 0)
    for k, v in over.items():
        setattr(a, k, v)
    return a


def _status(L, a):
    return L.vws_validate_sample_args(ctypes.byref(a))


def test_valid_args_pass(L):
    assert _status(L, _args(L)) == _lib.OK


@pytest.mark.parametrize("over,code,msg", [
    (dict(logits=None), _lib.ERR_INVALID_ARGUMENT, "logits is NULL"),
    (dict(batch=0), _lib.ERR_INVALID_ARGUMENT, "batch"),
    (dict(vocab=0), _lib.ERR_LIMIT, "vocab"),
    (dict(vocab=(1 << 19) + 1, logits_row_stride=(1 << 19) + 1), _lib.ERR_LIMIT, "vocab"),
    (dict(dtype=7), _lib.ERR_UNSUPPORTED_DTYPE, "dtype"),
    (dict(logits_row_stride=999), _lib.ERR_INVALID_ARGUMENT, "stride"),
    (dict(sampled=None), _lib.ERR_INVALID_ARGUMENT, "sampled"),
    (dict(uniforms=None), _lib.ERR_INVALID_ARGUMENT, "uniforms"),
    (dict(uniforms_row_stride=10), _lib.ERR_INVALID_ARGUMENT, "uniforms_row_stride"),
    (dict(num_logprobs=65), _lib.ERR_LIMIT, "num_logprobs"),
    (dict(num_logprobs=-2), _lib.ERR_LIMIT, "num_logprobs"),
    (dict(num_logprobs=5), _lib.ERR_INVALID_ARGUMENT, "logprob outputs"),
    (dict(prompt_ids=FAKE, prompt_width=-1), _lib.ERR_INVALID_ARGUMENT, "prompt_width"),
    (dict(output_ids=FAKE, output_width=8, output_row_stride=4), _lib.ERR_INVALID_ARGUMENT,
     "output_row_stride"),
    (dict(HIST, workspace=None), _lib.ERR_WORKSPACE_TOO_SMALL, "workspace"),
    (dict(HIST, workspace_bytes=256), _lib.ERR_WORKSPACE_TOO_SMALL, "workspace"),
    (dict(HIST, workspace=0x100010, workspace_bytes=1 << 20), _lib.ERR_INVALID_ARGUMENT, "aligned"),
    (dict(struct_size=8), _lib.ERR_INVALID_ARGUMENT, "struct_size"),
    (dict(adjust_ids=FAKE, adjust_width=4, adjust_row_stride=4), _lib.ERR_INVALID_ARGUMENT,
     "adjust_vals"),
    (dict(adjust_ids=FAKE, adjust_vals=FAKE, adjust_width=8, adjust_row_stride=4),
     _lib.ERR_INVALID_ARGUMENT, "adjust_row_stride"),
    (dict(allowed_mask=FAKE, allowed_row_stride=31), _lib.ERR_INVALID_ARGUMENT, "allowed_row_stride"),
    (dict(logit_softcap=-1.0), _lib.ERR_INVALID_ARGUMENT, "logit_softcap"),
    (dict(logit_softcap=float("nan")), _lib.ERR_INVALID_ARGUMENT, "logit_softcap"),
    (dict(logit_softcap=float("inf")), _lib.ERR_INVALID_ARGUMENT, "logit_softcap"),
    (dict(token_state=FAKE, token_state_row_stride=999), _lib.ERR_INVALID_ARGUMENT,
     "token_state_row_stride"),
    (dict(HIST, token_state=FAKE, token_state_row_stride=1000), _lib.ERR_INVALID_ARGUMENT,
     "token_state replaces"),
    (dict(token_state=FAKE, token_state_row_stride=1000, token_state_bits=FAKE,
          token_state_bits_stride=31), _lib.ERR_INVALID_ARGUMENT, "token_state_bits_stride"),
    (dict(token_state_bits=FAKE, token_state_bits_stride=32), _lib.ERR_INVALID_ARGUMENT,
     "without token_state"),
])
def test_invalid_args_rejected(L, over, code, msg):
    assert _status(L, _args(L, **over)) == code
    assert msg in _lib.last_error()


def test_history_grows_the_required_workspace(L):
    a = _args(L, output_ids=FAKE, output_width=512, output_row_stride=512)
    assert _status(L, a) == _lib.ERR_WORKSPACE_TOO_SMALL
    a.workspace_bytes = L.vws_sample_workspace_size(4, 1000, 512)
    assert _status(L, a) == _lib.OK


def test_processor_lists_grow_the_required_workspace(L):
    a = _args(L, adjust_ids=FAKE, adjust_vals=FAKE, adjust_width=100, adjust_row_stride=100)
    assert _status(L, a) == _lib.ERR_WORKSPACE_TOO_SMALL
    a.workspace_bytes = L.vws_sample_workspace_size(4, 1000, 100)
    assert _status(L, a) == _lib.OK
    assert _status(L, _args(L, allowed_mask=FAKE, allowed_row_stride=32)) == _lib.OK


def test_workspace_optional_without_history(L):
    """Without a history the workspace only carries the cooperative region: NULL or a smaller
    one is accepted (the launch then runs without the shared passes); with a history the hash
    needs it."""
    assert _status(L, _args(L, workspace=None, workspace_bytes=0)) == _lib.OK
    c0 = L.vws_sample_workspace_size(4, 1000, 0)
    assert _status(L, _args(L, workspace_bytes=c0 - 256)) == _lib.OK
    assert _status(L, _args(L, workspace_bytes=c0)) == _lib.OK
    assert _status(L, _args(L, **HIST, workspace=None, workspace_bytes=0)) == _lib.ERR_WORKSPACE_TOO_SMALL


def test_penalties_without_history_touch_nothing(L):
    """vws_apply_penalties with no history returns before looking at the workspace."""
    assert L.vws_apply_penalties(FAKE, 4, 1000, 1000, None, None, None, None, 0, 0, None, None,
                                 0, 0, None, None, 0, None) == _lib.OK


def test_coop_wait_polls_hook(L):
    prev = L.vws_set_coop_wait_polls(0)
    try:
        assert prev >= 0
        assert L.vws_set_coop_wait_polls(-1) == -1
        assert "polls" in _lib.last_error()
        assert L.vws_set_coop_wait_polls(7) == 0
    finally:
        L.vws_set_coop_wait_polls(prev)


def test_single_pass_hook(L):
    prev = L.vws_set_single_pass(0)
    try:
        assert prev == 1
        assert L.vws_set_single_pass(2) == -1
        assert "enabled" in _lib.last_error()
        assert L.vws_set_single_pass(1) == 0
    finally:
        L.vws_set_single_pass(prev)


def test_trace_set_only_in_the_trace_build(L):
    """The product library refuses vws_trace_set; the trace build (same ABI, same exports)
    takes a buffer or turns recording off, and rejects a count without a buffer."""
    assert L.vws_trace_set(None, 0) == _lib.ERR_UNSUPPORTED
    assert "trace build" in _lib.last_error()
    if not os.path.exists(_lib.TRACE_LIB_PATH):
        subprocess.run(["make", "-s", "-j4", "-C", os.path.join(ROOT, "vllm_webgpu_amd", "csrc"),
                        "trace"], check=True)
    T = _lib.load(_lib.TRACE_LIB_PATH)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.TRACE_LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    assert set(_declared()) <= set(re.findall(r"\bT (vws_\w+)", out))
    assert T.vws_trace_set(None, 0) == _lib.OK
    assert T.vws_trace_set(None, 4) == _lib.ERR_INVALID_ARGUMENT
    assert T.vws_trace_set(ctypes.c_void_p(4096), -1) == _lib.ERR_INVALID_ARGUMENT
    assert T.vws_trace_set(None, 0) == _lib.OK


def test_greedy_batches_need_no_uniforms(L):
    assert _status(L, _args(L, temperature=None, uniforms=None)) == _lib.OK


def test_launch_key_replaces_uniforms(L):
    """A by-value key for the launch stands in for uniforms or per-row keys."""
    assert _status(L, _args(L, uniforms=None, rng_key=0x1234, rng_key_set=1)) == _lib.OK
    assert _status(L, _args(L, uniforms=None, rng_key=0x1234, rng_key_set=0)) == _lib.ERR_INVALID_ARGUMENT
    assert "rng_key_set" in _lib.last_error()


def test_errors_raise_with_library_text(L):
    assert _status(L, _args(L, dtype=9)) != 0
    with pytest.raises(_lib.VwsError, match="unsupported logits dtype 9"):
        _lib.check(_lib.ERR_UNSUPPORTED_DTYPE)


def test_noalloc_checks_before_touching_the_device(L):
    """vws_sample_noalloc rejects bad arguments and batches beyond its static scratch on the
    host, before any device call (this test runs without a GPU)."""
    a = _args(L, output_ids=FAKE, output_width=2048, output_row_stride=2048, batch=4096)
    assert L.vws_sample_workspace_size(4096, 1000, 2048) > _lib.NOALLOC_SCRATCH_BYTES
    assert L.vws_sample_noalloc(ctypes.byref(a)) == _lib.ERR_LIMIT
    assert "static scratch" in _lib.last_error()
    assert L.vws_sample_noalloc(ctypes.byref(_args(L, **HIST, logits=None))) == _lib.ERR_INVALID_ARGUMENT
    assert "logits is NULL" in _lib.last_error()
    assert L.vws_sample_noalloc(ctypes.byref(_args(L, **HIST, struct_size=8))) == _lib.ERR_INVALID_ARGUMENT


def test_token_state_args(L):
    """The table replaces the lists: valid without a history list (and without a workspace),
    and its maintenance entry point checks its arguments on the host."""
    assert _status(L, _args(L, token_state=FAKE, token_state_row_stride=1000, workspace=None,
                            workspace_bytes=0)) == _lib.OK
    assert _status(L, _args(L, token_state=FAKE, token_state_row_stride=1000, token_state_bits=FAKE,
                            token_state_bits_stride=32, workspace=None, workspace_bytes=0)) == _lib.OK
    up = L.vws_token_state_update
    assert up(None, 1000, None, 0, 1000, 1, None, 0, FAKE, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert up(FAKE, 999, None, 0, 1000, 1, None, 0, FAKE, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert "row_stride" in _lib.last_error()
    assert up(FAKE, 1000, FAKE, 31, 1000, 1, None, 0, FAKE, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert "bits_stride" in _lib.last_error()
    assert up(FAKE, 1000, None, 0, 1000, 1, None, 0, FAKE, 2, None) == _lib.ERR_INVALID_ARGUMENT
    assert "kind" in _lib.last_error()
    assert up(FAKE, 1000, None, 0, 1000, 1, None, -1, FAKE, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert up(FAKE, 1000, None, 0, 1000, 1, None, 0, None, 0, None) == _lib.ERR_INVALID_ARGUMENT
    assert up(FAKE, 1000, None, 0, 0, 1, None, 0, FAKE, 0, None) == _lib.ERR_LIMIT
    assert up(FAKE, 1000, FAKE, 32, 1000, 0, None, 0, None, 0, None) == _lib.OK   # nothing to do

"""ctypes binding of the gfx950 sampler library ``vllm_webgpu_amd/_vws.so``.

The library's C ABI is declared in ``include/vws_sampler.h``; this module mirrors it one to one
(argument order, struct layout, status codes).  torch is imported before the library is loaded
so that the library binds to the HIP runtime torch already has in the process (both carry the
SONAME ``libamdhip64.so.7``).  A missing library is an error: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_vws.so")
# the same kernels built with per-workgroup phase stamps (vws_trace_set; vllm_webgpu_amd/trace.py)
TRACE_LIB_PATH = os.path.join(_HERE, "_vws_trace.so")

ABI_VERSION = 8
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED_DTYPE = 2
ERR_WORKSPACE_TOO_SMALL = 3
ERR_HIP = 4
ERR_LIMIT = 5
ERR_UNSUPPORTED = 6

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

FLAG_TOPP_NEAR_TIE = 0x1
FLAG_RACE_NEAR_TIE = 0x2
FLAG_DEGENERATE = 0x4
FLAG_GREEDY = 0x8
FLAG_GENERAL_PATH = 0x100
FLAG_STREAM_TOPP = 0x200
FLAG_TOPP_RECOUNT = 0x400
FLAG_TOPP_WIDE = 0x800

MAX_VOCAB = 1 << 19
MAX_LOGPROBS = 64
TOPK_MAX = 256
NOALLOC_SCRATCH_BYTES = 16 << 20
STATE_OUTPUT = 0
STATE_PROMPT = 1
STATE_PROMPT_FLAG = 0x80000000

TRACE_SLOTS = 16
(TRACE_ENTRY, TRACE_PARAMS, TRACE_FIRST, TRACE_SEED, TRACE_STREAM, TRACE_ROW, TRACE_EXIT,
 TRACE_WAVE_LOOP, TRACE_WAVE_PACK, TRACE_TP_HIST, TRACE_TP_MASS, TRACE_TP_CUT, TRACE_TP_RACE,
 TRACE_TP_LOGPROBS) = range(14)
TRACE_XCC = 14
TRACE_ROWID = 15

EXPORTED = (
    "vws_abi_version", "vws_last_error", "vws_sample_workspace_size", "vws_workspace_init",
    "vws_validate_sample_args", "vws_sample", "vws_sample_noalloc", "vws_argmax",
    "vws_topk_workspace_size",
    "vws_topk", "vws_softmax", "vws_apply_penalties", "vws_math_selftest",
    "vws_profile_begin", "vws_profile_end", "vws_set_coop_wait_polls", "vws_set_single_pass",
    "vws_token_state_update", "vws_trace_set",
)

KERNEL_KINDS = ("sample", "topk", "argmax", "softmax", "penalties", "other")

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32
_SZ = ctypes.c_size_t


class SampleArgs(ctypes.Structure):
    """Mirror of ``vws_sample_args``."""

    _fields_ = [
        ("struct_size", _U32), ("batch", _I32), ("vocab", _I32), ("dtype", _I32),
        ("logits", _P), ("logits_row_stride", _I64), ("logit_softcap", ctypes.c_float),
        ("logit_softcap_f16", _I32),
        ("temperature", _P), ("top_k", _P), ("top_p", _P), ("min_p", _P),
        ("repetition_penalty", _P), ("presence_penalty", _P), ("frequency_penalty", _P),
        ("prompt_ids", _P), ("prompt_row_stride", _I64), ("prompt_width", _I32), ("prompt_lens", _P),
        ("output_ids", _P), ("output_row_stride", _I64), ("output_width", _I32), ("output_lens", _P),
        ("token_state", _P), ("token_state_row_stride", _I64), ("token_state_rows", _P),
        ("token_state_bits", _P), ("token_state_bits_stride", _I64),
        ("allowed_mask", _P), ("allowed_row_stride", _I64),
        ("adjust_ids", _P), ("adjust_vals", _P), ("adjust_row_stride", _I64), ("adjust_width", _I32),
        ("adjust_lens", _P),
        ("uniforms", _P), ("uniforms_row_stride", _I64), ("rng_seeds", _P), ("rng_offsets", _P),
        ("rng_key", ctypes.c_uint64), ("rng_key_set", _I32),
        ("sampled", _P), ("row_flags", _P), ("num_kept", _P),
        ("num_logprobs", _I32), ("logprob_ids", _P), ("logprob_vals", _P), ("logprob_ranks", _P),
        ("workspace", _P), ("workspace_bytes", _SZ), ("stream", _P),
    ]


class VwsError(RuntimeError):
    """Raised when a library entry point returns a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"vws status {status}: {message}")
        self.status = status


_lock = threading.Lock()
_lib = None


def _declare(L):
    L.vws_abi_version.restype = _I32
    L.vws_abi_version.argtypes = []
    L.vws_last_error.restype = ctypes.c_char_p
    L.vws_last_error.argtypes = []
    L.vws_sample_workspace_size.restype = _SZ
    L.vws_sample_workspace_size.argtypes = [_I32, _I32, _I32]
    L.vws_workspace_init.restype = ctypes.c_int
    L.vws_workspace_init.argtypes = [_P, _SZ, _P]
    L.vws_validate_sample_args.restype = ctypes.c_int
    L.vws_validate_sample_args.argtypes = [ctypes.POINTER(SampleArgs)]
    L.vws_sample.restype = ctypes.c_int
    L.vws_sample.argtypes = [ctypes.POINTER(SampleArgs)]
    L.vws_sample_noalloc.restype = ctypes.c_int
    L.vws_sample_noalloc.argtypes = [ctypes.POINTER(SampleArgs)]
    L.vws_argmax.restype = ctypes.c_int
    L.vws_argmax.argtypes = [_P, _I32, _I32, _I32, _I64, _P, _P]
    L.vws_topk_workspace_size.restype = _SZ
    L.vws_topk_workspace_size.argtypes = [_I32, _I32, _I32]
    L.vws_topk.restype = ctypes.c_int
    L.vws_topk.argtypes = [_P, _I32, _I32, _I32, _I64, _I32, _P, _P, _P, _SZ, _P]
    L.vws_softmax.restype = ctypes.c_int
    L.vws_softmax.argtypes = [_P, _I32, _I32, _I32, _I64, _P, _P, _P, _P, _P]
    L.vws_apply_penalties.restype = ctypes.c_int
    L.vws_apply_penalties.argtypes = [_P, _I32, _I32, _I64, _P, _P, _P, _P, _I64, _I32, _P, _P,
                                      _I64, _I32, _P, _P, _SZ, _P]
    L.vws_math_selftest.restype = ctypes.c_int
    L.vws_math_selftest.argtypes = [_I32, _U32, _U32, _P, _P]
    L.vws_profile_begin.restype = ctypes.c_int
    L.vws_profile_begin.argtypes = [_I32]
    L.vws_profile_end.restype = ctypes.c_int
    L.vws_profile_end.argtypes = [_P, _P]
    L.vws_set_coop_wait_polls.restype = _I32
    L.vws_set_coop_wait_polls.argtypes = [_I32]
    L.vws_set_single_pass.restype = _I32
    L.vws_set_single_pass.argtypes = [_I32]
    L.vws_trace_set.restype = ctypes.c_int
    L.vws_trace_set.argtypes = [_P, _I32]
    L.vws_token_state_update.restype = ctypes.c_int
    L.vws_token_state_update.argtypes = [_P, _I64, _P, _I64, _I32, _I32, _P, _I32, _P, _I32, _P]


def load(path: str) -> ctypes.CDLL:
    """Loads a build of the library (after torch), declares it and checks its ABI version."""
    import torch  # noqa: F401  (HIP runtime first, see module docstring)

    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built: run `make -C vllm_webgpu_amd/csrc` (`... trace` for the trace "
            "build) or `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(path)
    _declare(L)
    v = L.vws_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"{os.path.basename(path)} ABI version {v} != {ABI_VERSION}")
    return L


def lib() -> ctypes.CDLL:
    """The library every entry point of this package calls: _vws.so, loaded on first use (or the
    build `use()` selected); raises if it is not built."""
    global _lib
    with _lock:
        if _lib is None:
            _lib = load(LIB_PATH)
    return _lib


class use:
    """``with _lib.use(path):`` makes the package's entry points call that build of the library
    (the trace build, say) inside the block, in this thread and every other."""

    def __init__(self, path: str):
        self.L = load(path)

    def __enter__(self) -> ctypes.CDLL:
        global _lib
        with _lock:
            self.prev, _lib = _lib, self.L
        return self.L

    def __exit__(self, *exc) -> None:
        global _lib
        with _lock:
            _lib = self.prev


def last_error() -> str:
    return lib().vws_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    if status != OK:
        raise VwsError(status, last_error())

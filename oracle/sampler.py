"""CPU oracle for the MI355X token-sampling path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker; the product package ``vllm_webgpu_amd`` never does.

It is a numpy/ctypes front end over ``oracle/vws_oracle.c`` (built into ``oracle/liboracle.so``
by ``oracle/Makefile``), which restates the sampling semantics row by row:

* greedy argmax with lowest-index ties -- ``vllm_webgpu/v1/model_runner.py:145``;
* the vLLM-v1 Sampler flow the plugin hands sampling to
  (``docs/superpowers/specs/2026-06-29-vllm-webgpu-design.md:451``): penalties, temperature,
  min-p, top-k, top-p, exponential race, raw logprobs;
* the WGSL kernels' contracts: ``shaders/generic/argmax.wgsl:1-60``,
  ``topk256.wgsl:1-70``, ``softmax.wgsl:1-71``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lock = threading.Lock()
_lib = None

FLAG_TOPP_NEAR_TIE = 0x1
FLAG_RACE_NEAR_TIE = 0x2
FLAG_DEGENERATE = 0x4
FLAG_GREEDY = 0x8

PARAMS_DTYPE = np.dtype(
    [("temperature", "<f4"), ("top_p", "<f4"), ("min_p", "<f4"), ("rep", "<f4"),
     ("pres", "<f4"), ("freq", "<f4"), ("top_k", "<i4"), ("_pad", "<i4")])
ROW_OUT_DTYPE = np.dtype(
    [("token", "<i4"), ("flags", "<u4"), ("n_kept", "<i4"), ("n_topk", "<i4"),
     ("mass_total", "<u8"), ("threshold", "<u8"), ("row_max", "<f4"), ("kth_y", "<f4")])


def build() -> str:
    """Compiles liboracle.so from vws_oracle.c with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            src = os.path.join(_HERE, "vws_oracle.c")
            if (not os.path.exists(_LIB_PATH)
                    or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src)):
                build()
            L = ctypes.CDLL(_LIB_PATH)
            P = ctypes.c_void_p
            L.vwo_exp.argtypes = [ctypes.c_float]
            L.vwo_exp.restype = ctypes.c_float
            L.vwo_log.argtypes = [ctypes.c_float]
            L.vwo_log.restype = ctypes.c_float
            L.vwo_mass.argtypes = [ctypes.c_float]
            L.vwo_mass.restype = ctypes.c_uint64
            L.vwo_key.argtypes = [ctypes.c_float]
            L.vwo_key.restype = ctypes.c_uint32
            L.vwo_scale_floor.argtypes = [ctypes.c_float, ctypes.c_uint64]
            L.vwo_scale_floor.restype = ctypes.c_uint64
            L.vwo_sample_batch.argtypes = [P, ctypes.c_int, ctypes.c_int, P, ctypes.c_int, P, P,
                                           ctypes.c_int, P, P, ctypes.c_int, P, P, ctypes.c_int,
                                           P, P, P, ctypes.c_int, P, P, P, P, ctypes.c_float,
                                           ctypes.c_int]
            L.vwo_softcap_row.argtypes = [P, ctypes.c_int, ctypes.c_float, ctypes.c_int, P]
            L.vwo_philox4x32_10.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32]
            L.vwo_philox_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32]
            L.vwo_philox_uniform.restype = ctypes.c_float
            L.vwo_philox_uniforms.argtypes = [P, P, ctypes.c_int, ctypes.c_int, P]
            L.vwo_check_round_f16.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_uint32, P, P]
            L.vwo_round_f16.argtypes = [ctypes.c_float]
            L.vwo_round_f16.restype = ctypes.c_float
            L.vwo_apply_adjustments_row.argtypes = [P, ctypes.c_int, P, P, P, ctypes.c_int]
            L.vwo_apply_penalties_row.argtypes = [P, ctypes.c_int, P, ctypes.c_int, P, ctypes.c_int,
                                                  ctypes.c_float, ctypes.c_float, ctypes.c_float]
            L.vwo_argmax_row.argtypes = [P, ctypes.c_int]
            L.vwo_argmax_row.restype = ctypes.c_int32
            L.vwo_topk_row.argtypes = [P, ctypes.c_int, ctypes.c_int, P, P]
            L.vwo_softmax_row.argtypes = [P, ctypes.c_int, ctypes.c_float, P, P, P]
            L.vwo_check_softcap.argtypes = [ctypes.c_float, ctypes.c_float, P, P, P, P, P]
            for name in ("vwo_check_exp", "vwo_check_log"):
                getattr(L, name).argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_uint32,
                                             P, P, P, P]
            _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bfloat16 bit patterns (uint16) to float32."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even narrowing of float32 to bfloat16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


# ---- scalar arithmetic (for pinning tests) ------------------------------------------------

def exp_det(d: float) -> float:
    return float(lib().vwo_exp(d))


def log_det(u: float) -> float:
    return float(lib().vwo_log(u))


def mass(e: float) -> int:
    return int(lib().vwo_mass(e))


def key(x: float) -> int:
    return int(lib().vwo_key(x))


def scale_floor(q: float, W: int) -> int:
    return int(lib().vwo_scale_floor(q, W))


def check_exp(lo: float, hi: float, stride: int = 1):
    return _check("vwo_check_exp", lo, hi, stride)


def check_log(lo: float, hi: float, stride: int = 1):
    return _check("vwo_check_log", lo, hi, stride)


def check_softcap(lo: float, hi: float):
    """vwo_softcap at cap 1 on every fp32 of [lo, hi]: max_err (absolute, against tanh in
    double), hash and count (as check_exp) and max_drop (largest max_{x' <= x} t(x') - t(x))."""
    me, w, d = ctypes.c_double(), ctypes.c_float(), ctypes.c_double()
    h, c = ctypes.c_uint64(), ctypes.c_uint64()
    lib().vwo_check_softcap(ctypes.c_float(lo), ctypes.c_float(hi), ctypes.byref(me),
                            ctypes.byref(w), ctypes.byref(h), ctypes.byref(c), ctypes.byref(d))
    return dict(max_err=me.value, worst=w.value, hash=h.value, count=c.value, max_drop=d.value)


def philox4x32_10(counter, key) -> list[int]:
    """Philox-4x32-10 of a 4-word counter under a 2-word key: the 4 output words."""
    c = np.ascontiguousarray(np.asarray(counter, np.uint32))
    assert c.shape == (4,)
    lib().vwo_philox4x32_10(_ptr(c), int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF)
    return [int(v) for v in c]


def philox_uniforms(seeds: np.ndarray, V: int, offsets: np.ndarray | None = None) -> np.ndarray:
    """The uniforms [B, V] the device generates from per-row 64-bit seeds (and offsets)."""
    sd = np.ascontiguousarray(np.asarray(seeds).astype(np.uint64))
    off = None if offsets is None else np.ascontiguousarray(np.asarray(offsets).astype(np.uint64))
    out = np.empty((sd.shape[0], V), np.float32)
    lib().vwo_philox_uniforms(_ptr(sd), _ptr(off), sd.shape[0], V, _ptr(out))
    return out


def check_round_f16(lo: float, hi: float, stride: int = 1):
    """vwo_round_f16 on every fp32 of [lo, hi]: hash and count (as check_exp)."""
    h, c = ctypes.c_uint64(), ctypes.c_uint64()
    lib().vwo_check_round_f16(lo, hi, stride, ctypes.byref(h), ctypes.byref(c))
    return dict(hash=h.value, count=c.value)


def _check(name, lo, hi, stride):
    mu, w = ctypes.c_int64(), ctypes.c_float()
    h, c = ctypes.c_uint64(), ctypes.c_uint64()
    getattr(lib(), name)(lo, hi, stride, ctypes.byref(mu), ctypes.byref(w), ctypes.byref(h),
                         ctypes.byref(c))
    return dict(max_ulp=mu.value, worst=w.value, hash=h.value, count=c.value)


# ---- row ops ----------------------------------------------------------------------------

def argmax(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    return np.array([lib().vwo_argmax_row(_ptr(r), r.shape[0]) for r in x], dtype=np.int32)


def topk(x: np.ndarray, k: int):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    vals = np.zeros((x.shape[0], k), np.float32)
    ids = np.zeros((x.shape[0], k), np.int32)
    for b in range(x.shape[0]):
        lib().vwo_topk_row(_ptr(x[b]), x.shape[1], k, _ptr(vals[b]), _ptr(ids[b]))
    return vals, ids


def softmax(x: np.ndarray, temperature: float = 1.0):
    """Returns (probs [B,V] f32, row_max [B] f32, log_sum [B] f64) with the sampler's exp."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    B, V = x.shape
    probs = np.zeros((B, V), np.float32)
    rm = np.zeros(B, np.float32)
    ls = np.zeros(B, np.float64)
    for b in range(B):
        lib().vwo_softmax_row(_ptr(x[b]), V, temperature, _ptr(probs[b]), _ptr(rm[b:b + 1]),
                              _ptr(ls[b:b + 1]))
    return probs, rm, ls


def apply_adjustments(x: np.ndarray, allowed=None, adjust_ids=None, adjust_vals=None) -> np.ndarray:
    """Copy of x [B,V] after the logits processors (allowed bitmask, bans, logit bias)."""
    x = np.array(x, dtype=np.float32, copy=True).reshape(-1, x.shape[-1])
    B, V = x.shape
    al = None if allowed is None else np.ascontiguousarray(allowed, np.uint32)
    ai = None if adjust_ids is None else np.ascontiguousarray(adjust_ids, np.int32)
    av = None if adjust_vals is None else np.ascontiguousarray(adjust_vals, np.float32)
    for b in range(B):
        lib().vwo_apply_adjustments_row(_ptr(x[b]), V, None if al is None else _ptr(al[b]),
                                        None if ai is None else _ptr(ai[b]),
                                        None if av is None else _ptr(av[b]),
                                        0 if ai is None else ai.shape[1])
    return x


def apply_penalties(x: np.ndarray, prompt_ids=None, output_ids=None, repetition=1.0,
                    presence=0.0, frequency=0.0) -> np.ndarray:
    """Penalised copy of x [B,V]; *_ids: padded int32 [B, W] (ids outside [0,V) are padding)."""
    x = np.array(x, dtype=np.float32, copy=True).reshape(-1, x.shape[-1])
    B, V = x.shape
    rep = np.broadcast_to(np.asarray(repetition, np.float32), (B,))
    pres = np.broadcast_to(np.asarray(presence, np.float32), (B,))
    freq = np.broadcast_to(np.asarray(frequency, np.float32), (B,))
    pr = None if prompt_ids is None else np.ascontiguousarray(prompt_ids, np.int32)
    out = None if output_ids is None else np.ascontiguousarray(output_ids, np.int32)
    for b in range(B):
        lib().vwo_apply_penalties_row(
            _ptr(x[b]), V, None if pr is None else _ptr(pr[b]), 0 if pr is None else pr.shape[1],
            None if out is None else _ptr(out[b]), 0 if out is None else out.shape[1],
            float(rep[b]), float(pres[b]), float(freq[b]))
    return x


def make_params(B, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition=1.0,
                presence=0.0, frequency=0.0) -> np.ndarray:
    p = np.zeros(B, PARAMS_DTYPE)
    p["temperature"] = temperature
    p["top_k"] = top_k
    p["top_p"] = top_p
    p["min_p"] = min_p
    p["rep"] = repetition
    p["pres"] = presence
    p["freq"] = frequency
    return p


def sample(logits: np.ndarray, params: np.ndarray, uniforms: np.ndarray | None = None,
           prompt_ids: np.ndarray | None = None, output_ids: np.ndarray | None = None,
           prompt_lens: np.ndarray | None = None, output_lens: np.ndarray | None = None,
           num_logprobs: int | None = None, allowed: np.ndarray | None = None,
           adjust_ids: np.ndarray | None = None, adjust_vals: np.ndarray | None = None,
           adjust_lens: np.ndarray | None = None, softcap: float | None = None,
           softcap_f16: bool = False) -> dict:
    """Samples every row of fp32 ``logits`` [B, V].

    ``params``: PARAMS_DTYPE [B] (see make_params).  ``uniforms``: fp32 [B, V] in (0, 1).
    History arrays: padded int32 [B, W]; ids outside [0, V) are padding (vLLM pads with V).
    Logits processors (before the penalties): ``allowed`` uint32 [B, ceil(V/32)] bitmask (bit
    set = allowed, None = all); ``adjust_ids`` int32 / ``adjust_vals`` fp32 [B, Wa]: value
    -inf bans the token, a finite value is added (logit bias).
    ``softcap`` > 0: the logits first go through Gemma's soft cap (see ``softcap_row``), each
    result rounded to f16 when ``softcap_f16``.
    Returns dict(token, flags, n_kept, n_topk, mass_total, threshold, row_max, kth_y,
    [lp_ids, lp_vals, ranks]).
    """
    x = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = x.shape
    assert params.dtype == PARAMS_DTYPE and params.shape == (B,)
    prm = np.ascontiguousarray(params)
    u = None if uniforms is None else np.ascontiguousarray(uniforms, np.float32)
    if u is None:
        u = np.full((B, V), 0.5, np.float32)
    pr = None if prompt_ids is None else np.ascontiguousarray(prompt_ids, np.int32)
    po = None if output_ids is None else np.ascontiguousarray(output_ids, np.int32)
    pl = None if prompt_lens is None else np.ascontiguousarray(prompt_lens, np.int32)
    ol = None if output_lens is None else np.ascontiguousarray(output_lens, np.int32)
    outs = np.zeros(B, ROW_OUT_DTYPE)
    L = -1 if num_logprobs is None else int(num_logprobs)
    lp_ids = lp_vals = ranks = None
    if L >= 0:
        lp_ids = np.zeros((B, L + 1), np.int32)
        lp_vals = np.zeros((B, L + 1), np.float32)
        ranks = np.zeros(B, np.int32)
    al = None if allowed is None else np.ascontiguousarray(allowed, np.uint32)
    ai = None if adjust_ids is None else np.ascontiguousarray(adjust_ids, np.int32)
    av = None if adjust_vals is None else np.ascontiguousarray(adjust_vals, np.float32)
    an = None if adjust_lens is None else np.ascontiguousarray(adjust_lens, np.int32)
    if ai is not None:
        assert av is not None and av.shape == ai.shape
    lib().vwo_sample_batch(_ptr(x), B, V, _ptr(pr), 0 if pr is None else pr.shape[1], _ptr(pl),
                           _ptr(po), 0 if po is None else po.shape[1], _ptr(ol),
                           _ptr(al), 0 if al is None else al.shape[1],
                           _ptr(ai), _ptr(av), 0 if ai is None else ai.shape[1], _ptr(an),
                           _ptr(prm), _ptr(u), L, _ptr(lp_ids), _ptr(lp_vals), _ptr(ranks),
                           _ptr(outs), float(softcap or 0.0), 1 if softcap_f16 else 0)
    res = {name: outs[name].copy() for name in ROW_OUT_DTYPE.names}
    if L >= 0:
        res.update(lp_ids=lp_ids, lp_vals=lp_vals, ranks=ranks)
    return res


def softcap_row(x: np.ndarray, cap: float, round_f16: bool = False) -> np.ndarray:
    """cap * tanh(x / cap) with the oracle's arithmetic (vwo_softcap), fp32 in and out; each
    result rounded to f16 and widened back when ``round_f16``."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().vwo_softcap_row(_ptr(x), x.size, float(cap), 1 if round_f16 else 0, _ptr(out))
    return out


def round_f16(x: float) -> float:
    """vwo_round_f16: fp32 -> binary16 (nearest, ties to even) -> fp32."""
    return lib().vwo_round_f16(float(x))

"""torch-facing wrappers of the gfx950 sampler library (device tensors in, device tensors out).

Every function enqueues work on torch's current HIP stream and returns without synchronising.
Inputs stay on the GPU; nothing here falls back to a CPU implementation -- if ``_vws.so`` is
missing or the tensors are not on a ROCm device, the call raises.

Reference interfaces these replace (paths under the vllm_webgpu reference):
``sample`` <- ``vllm_webgpu/v1/model_runner.py:139-166`` and ``run_inference.py:383-390``;
``argmax`` <- ``shaders/generic/argmax.wgsl``; ``topk`` <- ``shaders/generic/topk256.wgsl``;
``softmax`` <- ``shaders/generic/softmax.wgsl``.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass

import torch

from . import _lib

_ws_lock = threading.Lock()
_ws_cache: dict[int, torch.Tensor] = {}


def _stream_ptr() -> int:
    # the raw handle of the current stream, without building a Stream object
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device())


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if t.dtype == torch.float16:
        return _lib.DTYPE_F16
    raise TypeError(f"logits dtype {t.dtype} is not supported (float32, bfloat16 or float16)")


def _check_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a ROCm device tensor (got {t.device})")


def _row_param(x, B: int, dtype, device, name: str) -> torch.Tensor | None:
    if x is None:
        return None
    if not torch.is_tensor(x):
        x = torch.full((B,), x, dtype=dtype)
    if not (x.dtype == dtype and x.device == device and x.is_contiguous()):
        x = x.to(device=device, dtype=dtype).contiguous()
    if x.shape != (B,):
        raise ValueError(f"{name} must have shape ({B},), got {tuple(x.shape)}")
    return x


def _history(ids, lens, B: int, device, name: str):
    if ids is None:
        return None, 0, 0, None
    ids = ids.to(device=device, dtype=torch.int32)
    if ids.dim() != 2 or ids.shape[0] != B:
        raise ValueError(f"{name} must be [B, width] (got {tuple(ids.shape)})")
    if ids.stride(1) != 1:
        ids = ids.contiguous()
    if lens is not None:
        lens = lens.to(device=device, dtype=torch.int32).contiguous()
    return ids, ids.stride(0), ids.shape[1], lens


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Per-device scratch buffer, grown on demand and cleared once on the current stream.

    Calls that share a device share this buffer: run them in stream order (one stream), as the
    sampler kernels leave it clean for the next call but do not guard concurrent use.
    """
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        ws = _ws_cache.get(idx)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=f"cuda:{idx}")
            _lib.check(_lib.lib().vws_workspace_init(ws.data_ptr(), ws.numel(), _stream_ptr()))
            _ws_cache[idx] = ws
        return ws


@dataclass
class SampleResult:
    sampled: torch.Tensor                # [B] int32
    flags: torch.Tensor                  # [B] int32 (VWS_FLAG_* bits; uint32 on the device)
    num_kept: torch.Tensor               # [B] int32
    logprob_ids: torch.Tensor | None     # [B, L+1] int32
    logprob_vals: torch.Tensor | None    # [B, L+1] float32
    logprob_ranks: torch.Tensor | None   # [B] int32


class PreparedSample:
    """One ``vws_sample`` call with its arguments validated and packed once (``prepare_sample``):
    ``launch()`` issues it again on the current stream with one C call, reading the same input
    tensors (their current contents) and writing the same ``result`` tensors.  The object keeps
    every tensor it points at alive."""

    def __init__(self, args, result: SampleResult, keep: tuple):
        self.args = args
        self.result = result
        self._keep = keep

    def launch(self) -> SampleResult:
        self.args.stream = _stream_ptr()
        _lib.check(_lib.lib().vws_sample(ctypes.byref(self.args)))
        return self.result


def sample(logits: torch.Tensor, *args, **kwargs) -> SampleResult:
    """Samples one token per row of ``logits`` [B, V] (float32, bfloat16 or float16, on the
    GPU; each widened exactly to fp32).  Arguments: those of ``prepare_sample``."""
    return prepare_sample(logits, *args, **kwargs).launch()


def prepare_sample(logits: torch.Tensor, temperature=None, top_k=None, top_p=None, min_p=None,
                   repetition_penalty=None, presence_penalty=None, frequency_penalty=None,
                   prompt_ids=None, prompt_lens=None, output_ids=None, output_lens=None,
                   uniforms: torch.Tensor | None = None, num_logprobs: int | None = None,
                   allowed_mask: torch.Tensor | None = None, adjust_ids=None, adjust_vals=None,
                   adjust_lens=None, logit_softcap: float | None = None,
                   logit_softcap_f16: bool = False, rng_seeds: torch.Tensor | None = None,
                   rng_offsets: torch.Tensor | None = None, token_state: torch.Tensor | None = None,
                   token_state_rows: torch.Tensor | None = None,
                   token_state_bits: torch.Tensor | None = None,
                   rng_key: int | None = None) -> PreparedSample:
    """Validates and packs one sampling call over ``logits`` [B, V] (float32, bfloat16 or
    float16, on the GPU; each widened exactly to fp32) without launching it.

    Per-row parameters are scalars or [B] tensors; ``None`` means off (temperature None = every
    row greedy).  Histories are padded int32 [B, W] (ids outside [0, V) are padding).
    ``uniforms`` [B, V] float32 in (0, 1) drive the exponential race; instead, ``rng_seeds``
    [B] int64 (and optionally ``rng_offsets`` [B] int64) let the kernel generate them
    (Philox-4x32-10 keyed per row, evaluated only where a token races), or ``rng_key`` (a
    Python int) does for the whole launch: row r as with seed ``rng_key`` and offset r.  One of
    them is required whenever ``temperature`` is given.  Logits processors (before the
    penalties): ``allowed_mask`` int32 [B, ceil(V/32)] bit words (bit set = token allowed, see ``pack_allowed``), and the
    sparse ``adjust_ids`` int32 / ``adjust_vals`` float32 [B, W]: -inf bans a token, a finite
    value is added to its logit.  ``logit_softcap`` > 0: ``logits`` are the lm_head output
    before Gemma's final soft cap, which is applied first (cap * tanh(x / cap)); with
    ``logit_softcap_f16`` each capped value is rounded to float16 (the reference's shader
    stores the cap's output in an f16 buffer).  ``token_state`` int32 [R, >= V] (uint32 words,
    see ``token_state_update``) replaces ``prompt_ids``/``output_ids`` as the penalties' history;
    ``token_state_rows`` int32 [B] picks each row's table row (None = row i);
    ``token_state_bits`` int32 [R, >= ceil(V/32)], the table's bitmap of non-zero words (kept by
    ``token_state_update``), lets rows that top-p alone cuts keep the single-pass top-p path
    with their penalties.
    """
    _check_device(logits, "logits")
    cap = 0.0 if logit_softcap is None else float(logit_softcap)
    if not (cap >= 0.0) or cap == float("inf"):
        raise ValueError(f"logit_softcap must be finite and >= 0 (got {logit_softcap})")
    if logits.dim() != 2:
        raise ValueError("logits must be [B, V]")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    B, V = logits.shape
    dev = logits.device
    T = _row_param(temperature, B, torch.float32, dev, "temperature")
    K = _row_param(top_k, B, torch.int32, dev, "top_k")
    P = _row_param(top_p, B, torch.float32, dev, "top_p")
    MP = _row_param(min_p, B, torch.float32, dev, "min_p")
    R = _row_param(repetition_penalty, B, torch.float32, dev, "repetition_penalty")
    PR = _row_param(presence_penalty, B, torch.float32, dev, "presence_penalty")
    FR = _row_param(frequency_penalty, B, torch.float32, dev, "frequency_penalty")
    pid, pstride, pwidth, plens = _history(prompt_ids, prompt_lens, B, dev, "prompt_ids")
    oid, ostride, owidth, olens = _history(output_ids, output_lens, B, dev, "output_ids")
    aid, astride, awidth, alens = _history(adjust_ids, adjust_lens, B, dev, "adjust_ids")
    TS = TR = None
    if token_state is not None:
        _check_device(token_state, "token_state")
        if token_state.dtype != torch.int32 or token_state.dim() != 2 or token_state.stride(1) != 1:
            raise ValueError("token_state must be an int32 [rows, >= V] table with contiguous rows")
        if token_state.shape[1] < V:
            raise ValueError(f"token_state rows hold {token_state.shape[1]} words < vocab {V}")
        TS = token_state
        if token_state_bits is not None:
            _check_device(token_state_bits, "token_state_bits")
            if (token_state_bits.dtype != torch.int32 or token_state_bits.dim() != 2
                    or token_state_bits.stride(1) != 1):
                raise ValueError("token_state_bits must be an int32 [rows, >= ceil(V/32)] bitmap")
            if token_state_bits.shape[1] < (V + 31) // 32:
                raise ValueError(f"token_state_bits rows hold {token_state_bits.shape[1]} words < "
                                 f"ceil(vocab / 32) = {(V + 31) // 32}")
            if token_state_bits.shape[0] != token_state.shape[0]:
                raise ValueError("token_state_bits must have the table's rows")
        if token_state_rows is not None:
            TR = token_state_rows.to(device=dev, dtype=torch.int32).contiguous()
            if TR.shape != (B,):
                raise ValueError(f"token_state_rows must have shape ({B},)")
    aval = None
    if aid is not None:
        if adjust_vals is None:
            raise ValueError("adjust_vals is required with adjust_ids")
        aval = adjust_vals.to(device=dev, dtype=torch.float32)
        if aval.shape != aid.shape:
            raise ValueError(f"adjust_vals must have the shape of adjust_ids {tuple(aid.shape)}")
        if aval.stride() != aid.stride():
            aid, aval = aid.contiguous(), aval.contiguous()
            astride = aid.stride(0)
    AM = None
    if allowed_mask is not None:
        _check_device(allowed_mask, "allowed_mask")
        AM = allowed_mask.to(torch.int32)
        if AM.dim() != 2 or AM.shape[0] != B or AM.shape[1] < (V + 31) // 32:
            raise ValueError(f"allowed_mask must be [{B}, >= {(V + 31) // 32}] words")
        if AM.stride(1) != 1:
            AM = AM.contiguous()
    U = None
    if uniforms is not None:
        _check_device(uniforms, "uniforms")
        U = uniforms if uniforms.dtype == torch.float32 else uniforms.float()
        if U.stride(1) != 1:
            U = U.contiguous()
        if U.shape != (B, V):
            raise ValueError(f"uniforms must be [{B}, {V}]")
    SEED = OFF = None
    if rng_seeds is not None and U is None:
        SEED = _row_param(rng_seeds, B, torch.int64, dev, "rng_seeds")
        OFF = _row_param(rng_offsets, B, torch.int64, dev, "rng_offsets")
    if T is not None and U is None and SEED is None and rng_key is None:
        raise ValueError("uniforms, rng_seeds or rng_key is required when temperature is given")
    out3 = torch.empty((3, B), dtype=torch.int32, device=dev)  # one allocation for the three
    sampled, flags, nkept = out3[0], out3[1], out3[2]
    L = -1 if num_logprobs is None else int(num_logprobs)
    lp_ids = lp_vals = ranks = None
    if L >= 0:
        lp_ids = torch.empty((B, L + 1), dtype=torch.int32, device=dev)
        lp_vals = torch.empty((B, L + 1), dtype=torch.float32, device=dev)
        ranks = torch.empty(B, dtype=torch.int32, device=dev)
    L_lib = _lib.lib()
    nbytes = L_lib.vws_sample_workspace_size(B, V, pwidth + owidth + awidth)
    ws = workspace(nbytes, dev)
    a = _lib.SampleArgs()
    a.struct_size = ctypes.sizeof(_lib.SampleArgs)
    a.batch, a.vocab, a.dtype = B, V, _dtype_code(logits)
    a.logits, a.logits_row_stride = logits.data_ptr(), logits.stride(0)
    a.logit_softcap = cap
    a.logit_softcap_f16 = 1 if logit_softcap_f16 else 0
    a.temperature, a.top_k, a.top_p, a.min_p = _ptr(T), _ptr(K), _ptr(P), _ptr(MP)
    a.repetition_penalty, a.presence_penalty, a.frequency_penalty = _ptr(R), _ptr(PR), _ptr(FR)
    a.prompt_ids, a.prompt_row_stride, a.prompt_width, a.prompt_lens = _ptr(pid), pstride, pwidth, _ptr(plens)
    a.output_ids, a.output_row_stride, a.output_width, a.output_lens = _ptr(oid), ostride, owidth, _ptr(olens)
    if TS is not None:
        a.token_state, a.token_state_row_stride, a.token_state_rows = TS.data_ptr(), TS.stride(0), _ptr(TR)
        if token_state_bits is not None:
            a.token_state_bits, a.token_state_bits_stride = token_state_bits.data_ptr(), token_state_bits.stride(0)
    if AM is not None:
        a.allowed_mask, a.allowed_row_stride = AM.data_ptr(), AM.stride(0)
    if aid is not None:
        a.adjust_ids, a.adjust_vals = aid.data_ptr(), aval.data_ptr()
        a.adjust_row_stride, a.adjust_width, a.adjust_lens = astride, awidth, _ptr(alens)
    a.uniforms = _ptr(U)
    a.uniforms_row_stride = U.stride(0) if U is not None else 0
    a.rng_seeds, a.rng_offsets = _ptr(SEED), _ptr(OFF)
    if U is None and SEED is None and rng_key is not None:
        a.rng_key, a.rng_key_set = int(rng_key) & 0xFFFFFFFFFFFFFFFF, 1
    a.sampled, a.row_flags, a.num_kept = sampled.data_ptr(), flags.data_ptr(), nkept.data_ptr()
    a.num_logprobs = L
    a.logprob_ids, a.logprob_vals, a.logprob_ranks = _ptr(lp_ids), _ptr(lp_vals), _ptr(ranks)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    keep = (logits, T, K, P, MP, R, PR, FR, pid, plens, oid, olens, aid, aval, alens, TS, TR,
            token_state_bits, AM, U, SEED, OFF, ws)
    return PreparedSample(a, SampleResult(sampled, flags, nkept, lp_ids, lp_vals, ranks), keep)


def token_state_update(state: torch.Tensor, tokens: torch.Tensor, rows=None, prompt: bool = False,
                       vocab: int | None = None, bits: torch.Tensor | None = None) -> None:
    """Counts ``tokens`` (int32 [n] on the device) as output occurrences in the token-state
    table ``state`` (int32 [R, >= V], uint32 words: bit 31 prompt flag, low bits output count),
    or with ``prompt`` sets their prompt flags.  ``rows``: int32 [n] table rows, or one int for
    every id.  Ids outside [0, vocab) are padding (vocab defaults to the table's width).
    ``bits`` (int32 [R, >= ceil(V/32)]): the table's bitmap of non-zero words, whose bits of the
    updated ids are set."""
    _check_device(state, "state")
    if state.dtype != torch.int32 or state.dim() != 2 or state.stride(1) != 1:
        raise ValueError("state must be an int32 [rows, V] table with contiguous rows")
    V = state.shape[1] if vocab is None else int(vocab)
    if bits is not None:
        _check_device(bits, "bits")
        if bits.dtype != torch.int32 or bits.dim() != 2 or bits.stride(1) != 1:
            raise ValueError("bits must be an int32 [rows, >= ceil(V/32)] bitmap")
        if bits.shape[0] != state.shape[0] or bits.shape[1] < (V + 31) // 32:
            raise ValueError("bits must have the table's rows and >= ceil(V/32) words per row")
    tok = tokens.to(device=state.device, dtype=torch.int32).contiguous().view(-1)
    n = tok.numel()
    R = None
    row = 0
    if rows is None or isinstance(rows, int):
        row = 0 if rows is None else int(rows)
    else:
        R = rows.to(device=state.device, dtype=torch.int32).contiguous().view(-1)
        if R.numel() != n:
            raise ValueError(f"rows has {R.numel()} entries for {n} ids")
    kind = _lib.STATE_PROMPT if prompt else _lib.STATE_OUTPUT
    _lib.check(_lib.lib().vws_token_state_update(state.data_ptr(), state.stride(0), _ptr(bits),
                                                 bits.stride(0) if bits is not None else 0, V, n,
                                                 _ptr(R), row, tok.data_ptr(), kind, _stream_ptr()))


def pack_allowed(allowed: torch.Tensor) -> torch.Tensor:
    """bool [B, V] (True = allowed) -> int32 [B, ceil(V/32)] bit words, on the same device."""
    B, V = allowed.shape
    W = (V + 31) // 32
    bits = torch.zeros((B, W * 32), dtype=torch.int64, device=allowed.device)
    bits[:, :V] = allowed.to(torch.int64)
    weights = torch.bitwise_left_shift(torch.ones(32, dtype=torch.int64, device=allowed.device),
                                       torch.arange(32, device=allowed.device))
    words = (bits.view(B, W, 32) * weights).sum(dim=2)
    return (words - (words >= 2 ** 31).to(torch.int64) * 2 ** 32).to(torch.int32)


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """[B, V] -> [B] int32 argmax (lowest index on ties, NaN never selected)."""
    _check_device(logits, "logits")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    B, V = logits.shape
    out = torch.empty(B, dtype=torch.int32, device=logits.device)
    _lib.check(_lib.lib().vws_argmax(logits.data_ptr(), _dtype_code(logits), B, V, logits.stride(0),
                                     out.data_ptr(), _stream_ptr()))
    return out


def topk(logits: torch.Tensor, k: int):
    """[B, V] -> (values [B, k] float32, ids [B, k] int32), ordered (value desc, id asc)."""
    _check_device(logits, "logits")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    B, V = logits.shape
    vals = torch.empty((B, k), dtype=torch.float32, device=logits.device)
    ids = torch.empty((B, k), dtype=torch.int32, device=logits.device)
    L = _lib.lib()
    ws = workspace(L.vws_topk_workspace_size(B, V, k), logits.device)
    _lib.check(L.vws_topk(logits.data_ptr(), _dtype_code(logits), B, V, logits.stride(0), k,
                          vals.data_ptr(), ids.data_ptr(), ws.data_ptr(), ws.numel(), _stream_ptr()))
    return vals, ids


def softmax(logits: torch.Tensor, temperature=None):
    """softmax(x / T) per row -> (probs [B, V] f32, row_max [B] f32, log_sum [B] f32)."""
    _check_device(logits, "logits")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    B, V = logits.shape
    T = _row_param(temperature, B, torch.float32, logits.device, "temperature")
    probs = torch.empty((B, V), dtype=torch.float32, device=logits.device)
    rm = torch.empty(B, dtype=torch.float32, device=logits.device)
    ls = torch.empty(B, dtype=torch.float32, device=logits.device)
    _lib.check(_lib.lib().vws_softmax(logits.data_ptr(), _dtype_code(logits), B, V, logits.stride(0),
                                      _ptr(T), probs.data_ptr(), rm.data_ptr(), ls.data_ptr(),
                                      _stream_ptr()))
    return probs, rm, ls


def apply_penalties(logits: torch.Tensor, repetition_penalty=None, presence_penalty=None,
                    frequency_penalty=None, prompt_ids=None, prompt_lens=None, output_ids=None,
                    output_lens=None) -> torch.Tensor:
    """In-place vLLM-v1 penalties on float32 logits [B, V]; returns ``logits``."""
    _check_device(logits, "logits")
    if logits.dtype != torch.float32 or logits.stride(1) != 1:
        raise ValueError("apply_penalties needs contiguous-row float32 logits")
    B, V = logits.shape
    dev = logits.device
    R = _row_param(repetition_penalty, B, torch.float32, dev, "repetition_penalty")
    PR = _row_param(presence_penalty, B, torch.float32, dev, "presence_penalty")
    FR = _row_param(frequency_penalty, B, torch.float32, dev, "frequency_penalty")
    pid, pstride, pwidth, plens = _history(prompt_ids, prompt_lens, B, dev, "prompt_ids")
    oid, ostride, owidth, olens = _history(output_ids, output_lens, B, dev, "output_ids")
    L = _lib.lib()
    ws = workspace(L.vws_sample_workspace_size(B, V, pwidth + owidth), dev)
    _lib.check(L.vws_apply_penalties(logits.data_ptr(), B, V, logits.stride(0), _ptr(R), _ptr(PR),
                                     _ptr(FR), _ptr(pid), pstride, pwidth, _ptr(plens), _ptr(oid),
                                     ostride, owidth, _ptr(olens), ws.data_ptr(), ws.numel(),
                                     _stream_ptr()))
    return logits


def math_selftest(fn: int, key_lo: int, key_hi: int) -> tuple[int, int]:
    """Device hash of exp_det (fn=0), log_det (fn=1) or the soft cap's tanh (fn=2, cap 1) over
    an order-key range; synchronises."""
    out = torch.zeros(2, dtype=torch.int64, device="cuda")
    _lib.check(_lib.lib().vws_math_selftest(fn, key_lo, key_hi, out.data_ptr(), _stream_ptr()))
    h, c = out.cpu().tolist()
    return h & (2**64 - 1), c


def profile_begin(max_launches: int) -> None:
    """Records a hipEvent pair around each of the next ``max_launches`` library kernel launches."""
    _lib.check(_lib.lib().vws_profile_begin(max_launches))


def profile_end() -> dict:
    """Waits for the recorded events; returns {kind: (total_ms, launches)} and stops recording."""
    n = len(_lib.KERNEL_KINDS)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int32 * n)()
    _lib.check(_lib.lib().vws_profile_end(ctypes.cast(ms, ctypes.c_void_p),
                                          ctypes.cast(cnt, ctypes.c_void_p)))
    return {k: (ms[i], cnt[i]) for i, k in enumerate(_lib.KERNEL_KINDS) if cnt[i]}

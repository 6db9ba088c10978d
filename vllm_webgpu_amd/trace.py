"""Phase trace of the sampling kernel: per-workgroup clock stamps from the trace build of the
library (``_vws_trace.so``, ``vws_trace_set``), aggregated per phase and per XCD.

    python -m vllm_webgpu_amd.trace --config 3 [--launches 24] [--table-history]
                                    [--logprobs L] [--mask-rows N]

Runs ``--launches`` back-to-back ``vws_sample`` launches of one of the BASELINE workloads (three
input sets rotated, as ``bench.py`` does) after warm-up launches, each launch writing its own
records, and prints markdown tables:

* phases of a row, relative to its workgroup's first instruction, per path the row took
  (single pass, single-pass top-p path, multi-pass path): parameters read, first iteration of
  logits in the last wave, seed published, the last wave's own stream and pack, every wave streamed, row done,
  and the workgroup's help with other rows' passes after it;
* per XCD, relative to the launch's first workgroup: when its workgroups started, ended their
  streams and their rows;
* per launch: first start to last exit, next to the kernel's own duration from the
  kernel-stamped events of ``vws_profile_begin``.

The device clock (``s_memrealtime``) runs at 100 MHz: stamps resolve 0.01 us.  The trace build
adds a few stores per workgroup and nothing else; its kernel durations are within noise of the
product build's.
"""
from __future__ import annotations

import argparse
import sys

import numpy as np

from . import _lib

PATHS = {"single pass": lambda f: (f & (_lib.FLAG_GENERAL_PATH | _lib.FLAG_STREAM_TOPP)) == 0,
         "top-p path": lambda f: (f & _lib.FLAG_STREAM_TOPP) != 0,
         "multi-pass": lambda f: (f & _lib.FLAG_GENERAL_PATH) != 0}
TICKS_PER_US = 100.0


def _inputs(cfg: int, dev, table_history: bool, sets: int, logprobs=-1, mask_rows: int = 0):
    import torch

    from . import ops
    from . import workloads as W

    w = W.config(cfg)
    B, V = w.shape
    if w.dtype == "bf16":
        x = torch.from_numpy(w.logits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        x = torch.from_numpy(w.logits).to(dev)
    xs = [x] + [torch.roll(x, i, 0).contiguous() for i in range(1, sets)]
    greedy_all = bool(np.all(~(w.temperature >= np.float32(1e-5))))
    kw = dict(temperature=None if greedy_all else torch.from_numpy(w.temperature).to(dev),
              top_k=torch.from_numpy(w.top_k).to(dev), top_p=torch.from_numpy(w.top_p).to(dev),
              min_p=torch.from_numpy(w.min_p).to(dev),
              repetition_penalty=torch.from_numpy(w.repetition).to(dev),
              presence_penalty=torch.from_numpy(w.presence).to(dev),
              frequency_penalty=torch.from_numpy(w.frequency).to(dev),
              output_ids=None if w.output_ids is None else torch.from_numpy(w.output_ids).to(dev),
              uniforms=None if w.uniforms is None else torch.from_numpy(w.uniforms).to(dev),
              num_logprobs=w.num_logprobs)
    name = w.name
    if logprobs is None or logprobs >= 0:
        kw["num_logprobs"] = logprobs
        name += " (no logprobs)" if logprobs is None else f" ({logprobs} logprobs)"
    if mask_rows:
        # the first mask_rows rows restricted to 20 tokens each, the others allowed everything
        from . import ops

        allowed = torch.ones((B, V), dtype=torch.bool)
        rng = np.random.default_rng(62)
        for i in range(mask_rows):
            allowed[i] = False
            allowed[i, torch.from_numpy(rng.choice(V, 20, replace=False))] = True
        kw["allowed_mask"] = ops.pack_allowed(allowed.to(dev))
        name += f" ({mask_rows} masked rows)"
    if table_history:
        # the workload's history ids (or, without one, C3's penalties from a 512-token output
        # history per row) as the token-state table and its bitmap
        if w.output_ids is not None:
            hist = w.output_ids
        else:
            hist = np.random.default_rng(W.SEED_BASE + 35).integers(0, V, (B, 512)).astype(np.int32)
            kw.update(repetition_penalty=1.1, presence_penalty=0.5, frequency_penalty=0.3)
        st = torch.zeros((B, V), dtype=torch.int32, device=dev)
        bits = torch.zeros((B, (V + 31) // 32), dtype=torch.int32, device=dev)
        rows = torch.arange(B, dtype=torch.int32, device=dev).repeat_interleave(hist.shape[1])
        ops.token_state_update(st, torch.from_numpy(np.ascontiguousarray(hist)).to(dev).reshape(-1),
                               rows=rows, bits=bits)
        kw.update(output_ids=None, token_state=st, token_state_bits=bits)
        name += " (history from the token-state table)"
    return w, xs, kw, name


def collect(cfg: int, launches: int = 24, warmup: int = 10, sets: int = 3,
            table_history: bool = False, logprobs=-1, mask_rows: int = 0):
    """Runs the launches through the trace build, then the same sequence through the product
    build; returns (records [launches, B, slots] int64, flags [launches, B] uint32, (trace,
    product) kernel us per launch, workload name, batch)."""
    import torch

    from . import ops

    dev = torch.device("cuda:0")
    w, xs, kw, name = _inputs(cfg, dev, table_history, sets, logprobs, mask_rows)
    B = w.shape[0]
    # every launch prepared up front, so that the launches run back to back (a host that falls
    # behind would start each one from an idle device, which changes its timing)
    calls = [ops.prepare_sample(x, **kw) for x in xs]
    with _lib.use(_lib.TRACE_LIB_PATH) as L:
        for i in range(warmup):
            calls[i % sets].launch()
        torch.cuda.synchronize()
        buf = torch.zeros((launches, B, _lib.TRACE_SLOTS), dtype=torch.int64, device=dev)
        ops.profile_begin(launches + 8)
        try:
            for i in range(launches):
                _lib.check(L.vws_trace_set(buf[i].data_ptr(), B))
                calls[(warmup + i) % sets].launch()
            torch.cuda.synchronize()
        finally:
            _lib.check(L.vws_trace_set(None, 0))
            kern = ops.profile_end()
    # the same launch sequence on the product build, for the trace build's overhead
    for i in range(warmup):
        calls[i % sets].launch()
    torch.cuda.synchronize()
    ops.profile_begin(launches + 8)
    try:
        for i in range(launches):
            calls[(warmup + i) % sets].launch()
        torch.cuda.synchronize()
    finally:
        kprod = ops.profile_end()
    rec = buf.cpu().numpy()
    # each input set's flags (the same on every launch of the set: same inputs, same results)
    per_set = [c.result.flags.cpu().numpy().view(np.uint32) for c in calls]
    fl = np.stack([per_set[(warmup + i) % sets] for i in range(launches)])
    us = lambda k: k["sample"][0] / max(k["sample"][1], 1) * 1e3 if "sample" in k else float("nan")
    return rec, fl, (us(kern), us(kprod)), name, B


def _stats(v) -> str:
    v = np.asarray(v, float)
    if v.size == 0:
        return "| – | – | – | – |"
    return (f"| {np.median(v):.2f} | {np.percentile(v, 10):.2f} | {np.percentile(v, 90):.2f} "
            f"| {v.max():.2f} |")


def report(rec, fl, kernel_us, name: str, B: int) -> str:
    n_launch = rec.shape[0]
    kernel_us, product_us = kernel_us
    out = [f"## Phase trace: {name}", "",
           f"{n_launch} back-to-back launches of B = {B} rows; kernel-stamped duration "
           f"{kernel_us:.2f} us per launch of the trace build, {product_us:.2f} us of the product "
           "build on the same launch sequence (the difference is the stamps' cost).", ""]
    rowid = rec[:, :, _lib.TRACE_ROWID]
    rflags = np.take_along_axis(fl, np.clip(rowid, 0, B - 1), axis=1)  # flags of each WG's row
    ent = rec[:, :, _lib.TRACE_ENTRY]

    def rel(slot, base=None):
        """us from the workgroup's entry (base None) or from a slot of the same workgroup;
        NaN where the slot was not reached."""
        b = ent if base is None else rec[:, :, base]
        v = (rec[:, :, slot] - b) / TICKS_PER_US
        return np.where((rec[:, :, slot] > 0) & (b > 0), v, np.nan)

    phases = [("parameters read", rel(_lib.TRACE_PARAMS)),
              ("first iteration in the last wave", rel(_lib.TRACE_FIRST)),
              ("seed published", rel(_lib.TRACE_SEED)),
              ("the last wave examined its share", rel(_lib.TRACE_WAVE_LOOP)),
              ("the last wave packed its candidates", rel(_lib.TRACE_WAVE_PACK)),
              ("every wave streamed", rel(_lib.TRACE_STREAM)),
              ("row done", rel(_lib.TRACE_ROW)),
              ("finish: streamed -> row done", rel(_lib.TRACE_ROW, _lib.TRACE_STREAM)),
              ("  top-p: streamed -> history tokens buffered", rel(_lib.TRACE_TP_HIST, _lib.TRACE_STREAM)),
              ("  top-p: streamed -> exact masses in", rel(_lib.TRACE_TP_MASS, _lib.TRACE_STREAM)),
              ("  top-p: masses -> cut decided", rel(_lib.TRACE_TP_CUT, _lib.TRACE_TP_MASS)),
              ("  top-p: cut -> race done", rel(_lib.TRACE_TP_RACE, _lib.TRACE_TP_CUT)),
              ("  top-p: race -> raw logprobs done", rel(_lib.TRACE_TP_LOGPROBS, _lib.TRACE_TP_RACE)),
              ("  top-p: logprobs -> row done", rel(_lib.TRACE_ROW, _lib.TRACE_TP_LOGPROBS)),
              ("help after the row", rel(_lib.TRACE_EXIT, _lib.TRACE_ROW))]
    for pname, pick in PATHS.items():
        sel = pick(rflags)
        if not sel.any():
            continue
        out += [f"Rows on the {pname} ({int(sel.sum())} of {sel.size} workgroup records), us after "
                "the workgroup's first instruction:", "",
                "| phase | median | p10 | p90 | max |", "|---|---|---|---|---|"]
        for label, v in phases:
            vv = v[sel]
            vv = vv[np.isfinite(vv)]
            if vv.size:
                out.append(f"| {label} " + _stats(vv))
        out.append("")

    t0 = ent.min(axis=1, keepdims=True)
    L = lambda slot: np.where(rec[:, :, slot] > 0, (rec[:, :, slot] - t0) / TICKS_PER_US, np.nan)
    xcc = rec[:, :, _lib.TRACE_XCC]
    e, s, r, x = L(_lib.TRACE_ENTRY), L(_lib.TRACE_STREAM), L(_lib.TRACE_ROW), L(_lib.TRACE_EXIT)
    out += ["Per XCD, us after the launch's first workgroup started (medians over the launches of "
            "each launch's per-XCD figure):", "",
            "| XCD | WGs per launch | first start | last start | streams ended (median) | "
            "last stream end | rows done (median) | last row done | last exit |",
            "|---|---|---|---|---|---|---|---|---|"]
    for c in range(8):
        m = xcc == c
        if not m.any():
            continue

        def per_launch(a, fn):
            vals = [fn(a[i][m[i]]) for i in range(n_launch) if m[i].any() and np.isfinite(a[i][m[i]]).any()]
            return np.median(vals) if vals else np.nan

        out.append(f"| {c} | {m.sum() / n_launch:.0f} | {per_launch(e, np.nanmin):.2f} | "
                   f"{per_launch(e, np.nanmax):.2f} | {per_launch(s, np.nanmedian):.2f} | "
                   f"{per_launch(s, np.nanmax):.2f} | {per_launch(r, np.nanmedian):.2f} | "
                   f"{per_launch(r, np.nanmax):.2f} | {per_launch(x, np.nanmax):.2f} |")
    span = np.nanmax(x, axis=1)
    out += ["", f"Launch span, first start -> last exit: median {np.median(span):.2f} us, "
            f"min {span.min():.2f}, max {span.max():.2f} (kernel-stamped: {kernel_us:.2f} us; the "
            "difference is the dispatch before the first workgroup starts and the end of the "
            "kernel after the last one exits).",
            f"Start stagger, first -> last workgroup start: median "
            f"{np.median(np.nanmax(e, axis=1)):.2f} us.", ""]
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--launches", type=int, default=24)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--table-history", action="store_true",
                    help="the history as the token-state table and bitmap (C3's penalties for "
                         "workloads without a history)")
    ap.add_argument("--logprobs", type=int, default=-1,
                    help="raw logprobs per row (0..64) instead of the workload's; -2: none")
    ap.add_argument("--mask-rows", type=int, default=0,
                    help="an allowed mask with the first N rows restricted to 20 tokens")
    args = ap.parse_args(argv)
    lp = None if args.logprobs == -2 else args.logprobs
    rec, fl, kus, name, B = collect(args.config, args.launches, args.warmup,
                                    table_history=args.table_history, logprobs=lp,
                                    mask_rows=args.mask_rows)
    print(report(rec, fl, kus, name, B))
    return 0


if __name__ == "__main__":
    sys.exit(main())

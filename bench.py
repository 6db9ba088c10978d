#!/usr/bin/env python3
"""Benchmark of the MI355X token sampler on the headline workload (configuration 3).

C3: fp32 logits [B=256, V=128256] ~ N(0, 3); per row a 512-token prior-output history drives
repetition 1.1 / presence 0.5 / frequency 0.3 penalties; then temperature 0.7, top-k 50,
top-p 0.9 and caller-supplied uniforms (exponential race).  One "step" = one ``vws_sample``
call over the whole batch with inputs resident in HBM.  Three input sets (rolled copies, 394 MB
of logits) are rotated so re-reads cannot be served by the 256 MB MALL.

Prints ONE JSON line (rank 0): rows/s, ms per step, the HBM roofline of the dominant kernel
(algorithmic bytes / its average event-timed duration, peak 8 TB/s) and the CPU baseline (the
torch restatement of vLLM's sampler, oracle/vllm_torch.py, on a bounded sample of the rows).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0
METRIC = "sampled rows/sec + HBM GB/s (% peak), B=256 V=128256 top-k/top-p/penalties"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_args(lib_mod, logits, T, K, P, MP, R, PR, FR, hist, U, out, flags, nkept, ws,
               lp=None):
    """vws_sample_args over device tensors; ``hist``/``U`` may be None, ``lp`` = (L, ids, vals,
    ranks) requests logprobs."""
    import torch

    a = lib_mod.SampleArgs()
    a.struct_size = ctypes.sizeof(lib_mod.SampleArgs)
    B, V = logits.shape
    a.batch, a.vocab = B, V
    a.dtype = lib_mod.DTYPE_BF16 if logits.dtype == torch.bfloat16 else lib_mod.DTYPE_F32
    a.logits, a.logits_row_stride = logits.data_ptr(), logits.stride(0)
    all_greedy = bool((T < 1e-5).all())  # greedy batches pass no temperature (and no uniforms)
    a.temperature = None if all_greedy else T.data_ptr()
    a.top_k, a.top_p, a.min_p = K.data_ptr(), P.data_ptr(), MP.data_ptr()
    a.repetition_penalty, a.presence_penalty, a.frequency_penalty = R.data_ptr(), PR.data_ptr(), FR.data_ptr()
    if hist is not None:
        a.output_ids, a.output_row_stride, a.output_width = hist.data_ptr(), hist.stride(0), hist.shape[1]
    if U is not None:
        a.uniforms, a.uniforms_row_stride = U.data_ptr(), U.stride(0)
    a.sampled, a.row_flags, a.num_kept = out.data_ptr(), flags.data_ptr(), nkept.data_ptr()
    a.num_logprobs = -1
    if lp is not None:
        a.num_logprobs = lp[0]
        a.logprob_ids, a.logprob_vals, a.logprob_ranks = lp[1].data_ptr(), lp[2].data_ptr(), lp[3].data_ptr()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    return a


def timed_region(step, steps: int, stream, launches_per_step: int = 1, kernel_events: bool = True):
    """Runs ``step(i)`` for i < steps between two hipEvents on ``stream``; with
    ``kernel_events`` every library launch in between carries its own kernel-stamped event pair
    (vws_profile_begin).  Returns the raw figures: region ms, wall s, and per kernel kind the
    summed kernel ms and launches.  (The per-launch events cost host time and stretch the region
    by a few microseconds per launch, so the region that defines ms/step runs without them.)"""
    import torch

    from vllm_webgpu_amd import ops

    torch.cuda.synchronize()
    if kernel_events:
        ops.profile_begin(steps * launches_per_step + 8)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern = ops.profile_end() if kernel_events else {}
    return {"steps": steps, "region_ms": e0.elapsed_time(e1), "wall_s": wall,
            "kernels": {k: {"ms": v[0], "launches": v[1]} for k, v in kern.items()}}


def kernel_us(t, kind="sample"):
    k = t["kernels"].get(kind)
    return None if not k else k["ms"] / k["launches"] * 1e3


def v1_forward_timing(w, logits, T, K, P, MP, R, PR, FR, hist, dev, steps: int, warmup: int):
    """Sampler.forward (vLLM-v1 signature) on device-resident metadata: wall time per call
    (host work included, synchronised at both ends) and stream time per call (hipEvents)."""
    import torch

    from vllm_webgpu_amd.v1.sample.metadata import SamplingMetadata
    from vllm_webgpu_amd.v1.sample.sampler import Sampler

    greedy = ~(w.temperature >= np.float32(1e-5))
    m = SamplingMetadata(
        temperature=None if greedy.all() else T, all_greedy=bool(greedy.all()),
        all_random=not greedy.any(), top_p=P, top_k=K, generators={},
        max_num_logprobs=w.num_logprobs, no_penalties=hist is None, prompt_token_ids=None,
        frequency_penalties=FR, presence_penalties=PR, repetition_penalties=R,
        output_token_ids=[], min_p=MP, output_token_ids_tensor=hist)
    sampler = Sampler()
    for _ in range(warmup):
        sampler(logits, m)
    t = timed_region(lambda i: sampler(logits, m), steps, torch.cuda.current_stream(),
                     kernel_events=False)
    return {"wall_us": t["wall_s"] / steps * 1e6, "gpu_us": t["region_ms"] / steps * 1e3,
            "timing": t,
            "uniforms": "generated in the kernel (Philox-4x32-10, one key per row and step)"}


def history_free_timing(lib_mod, L, sets, T, K, P, MP, R, PR, FR, out, flags, nkept, ws, lp,
                        stream, steps: int, warmup: int) -> dict:
    """The sampling kernel on the same logits and uniforms with no history (penalties off)."""
    argv = []
    for lg, u, _ in sets:
        a = build_args(lib_mod, lg, T, K, P, MP, R, PR, FR, None, u, out, flags, nkept, ws, lp)
        a.stream = stream.cuda_stream
        argv.append(a)
    for i in range(warmup):
        lib_mod.check(L.vws_sample(ctypes.byref(argv[i % len(argv)])))
    return timed_region(lambda i: L.vws_sample(ctypes.byref(argv[i % len(argv)])), steps, stream)


def generated_timing(lib_mod, L, sets, T, K, P, MP, R, PR, FR, out, flags, nkept, ws, lp,
                     stream, B, steps: int, warmup: int) -> dict:
    """The sampling kernel alone with generated uniforms (keys instead of a [B, V] tensor)."""
    import torch

    dev = out.device
    seeds = torch.arange(1, B + 1, dtype=torch.int64, device=dev) * 0x9E3779B97F4A7C15 // 7
    argv = []
    for lg, _, h in sets:
        a = build_args(lib_mod, lg, T, K, P, MP, R, PR, FR, h, None, out, flags, nkept, ws, lp)
        a.rng_seeds = seeds.data_ptr()
        a.stream = stream.cuda_stream
        argv.append(a)
    for i in range(warmup):
        lib_mod.check(L.vws_sample(ctypes.byref(argv[i % len(argv)])))
    return timed_region(lambda i: L.vws_sample(ctypes.byref(argv[i % len(argv)])), steps, stream)


def token_state_timing(lib_mod, L, W, w, sets, T, K, P, MP, R, PR, FR, out, flags, nkept, ws, lp,
                       stream, steps: int, warmup: int) -> dict:
    """The sampling kernel with the penalties' history in a per-request token-state table
    instead of id lists: (a) C3's own 512-token output histories, (b) a 4096-token prompt plus a
    1024-token output per row (more distinct ids than the single pass's LDS hash holds), each
    checked against the oracle on the id lists for its first 16 rows."""
    import torch

    from oracle import sampler as O  # checker only

    B, V = w.shape
    res = {}
    for name, (prompt, outp) in (("c3_history", (None, w.output_ids)),
                                 ("long_history_4096_1024", W.long_history(w))):
        st = torch.from_numpy(W.token_state_table(B, V, prompt, outp).view(np.int32)).to(out.device)
        tabs = [st] + [torch.roll(st, shifts=i, dims=0).contiguous() for i in range(1, len(sets))]
        argv = []
        for (lg, u, _), tb in zip(sets, tabs):
            a = build_args(lib_mod, lg, T, K, P, MP, R, PR, FR, None, u, out, flags, nkept, ws, lp)
            a.token_state, a.token_state_row_stride = tb.data_ptr(), tb.stride(0)
            a.stream = stream.cuda_stream
            argv.append(a)
        lib_mod.check(L.vws_sample(ctypes.byref(argv[0])))
        torch.cuda.synchronize()
        n = 16
        got = out.cpu().numpy()[:n]
        gflags = flags.cpu().numpy().view(np.uint32)
        prm = O.make_params(n, w.temperature[:n], w.top_k[:n], w.top_p[:n], w.min_p[:n],
                            w.repetition[:n], w.presence[:n], w.frequency[:n])
        ref = O.sample(w.logits_f32()[:n], prm, w.uniforms[:n],
                       prompt_ids=None if prompt is None else prompt[:n], output_ids=outp[:n])
        for i in range(warmup):
            lib_mod.check(L.vws_sample(ctypes.byref(argv[i % len(argv)])))
        t = timed_region(lambda i: L.vws_sample(ctypes.byref(argv[i % len(argv)])), steps, stream)
        res[name] = {"kernel_us": kernel_us(t), "timing": t,
                     "parity_rows": n, "token_mismatches": int((got != ref["token"]).sum()),
                     "general_path_rows": int(((gflags & 0x100) != 0).sum()),
                     "history": {"prompt": 0 if prompt is None else int(prompt.shape[1]),
                                 "output": int(outp.shape[1])}}
    return res


def variant_timing(lib_mod, L, w, sets, T, K, P, MP, R, PR, FR, out, flags, nkept, ws, stream,
                   steps: int, warmup: int, num_logprobs=None, parity_rows: int = 16,
                   allowed=None, hist=None, table: bool = False, adjust=None) -> dict:
    """The launch with one thing changed (raw logprobs requested, an allowed mask [B, V] bool,
    a [B, H] output history replacing the workload's: as padded id lists, or with `table` as
    the token-state table and its bitmap the runner keeps, built by vws_token_state_update; or
    `adjust` = (ids, vals, lens), a sparse processor list), timed with kernel-stamped events and
    checked against the oracle on its first rows."""
    import torch

    from oracle import sampler as O  # checker only

    B, V = w.shape
    words = hist_d = None
    if allowed is not None:
        wb = np.zeros((B, (V + 31) // 32 * 32), np.uint64)
        wb[:, :V] = allowed
        words = (wb.reshape(B, -1, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)
        words_d = torch.from_numpy(words.view(np.int32)).to(out.device)
    if hist is not None:
        hist_d = torch.from_numpy(hist).to(out.device)
    state = bits = None
    if table:
        from vllm_webgpu_amd import ops

        state = torch.zeros((B, V), dtype=torch.int32, device=out.device)
        bits = torch.zeros((B, (V + 31) // 32), dtype=torch.int32, device=out.device)
        rows = torch.arange(B, dtype=torch.int32, device=out.device).repeat_interleave(hist.shape[1])
        ops.token_state_update(state, hist_d.reshape(-1), rows=rows, bits=bits)
        torch.cuda.synchronize()
    out_ids = w.output_ids if hist is None else hist
    lp = None
    if num_logprobs is not None:
        lp = (num_logprobs, torch.empty((B, num_logprobs + 1), dtype=torch.int32, device=out.device),
              torch.empty((B, num_logprobs + 1), dtype=torch.float32, device=out.device),
              torch.empty(B, dtype=torch.int32, device=out.device))
    argv, keep = [], []
    adj_d = None if adjust is None else tuple(torch.from_numpy(t).to(out.device) for t in adjust)
    for i, (lg, u, h) in enumerate(sets):
        trows = None
        if table:
            # the rotated set's row r has history row (r - i) mod B: the table's row map
            trows = torch.remainder(torch.arange(B, device=out.device) - i, B).to(torch.int32)
            keep.append(trows)
            h = None
        elif hist_d is not None:
            h = torch.roll(hist_d, shifts=i, dims=0).contiguous() if i else hist_d
            keep.append(h)
        a = build_args(lib_mod, lg, T, K, P, MP, R, PR, FR, h, u, out, flags, nkept, ws, lp)
        if table:
            a.token_state, a.token_state_row_stride = state.data_ptr(), state.stride(0)
            a.token_state_rows = trows.data_ptr()
            a.token_state_bits, a.token_state_bits_stride = bits.data_ptr(), bits.stride(0)
        if words is not None:
            a.allowed_mask, a.allowed_row_stride = words_d.data_ptr(), words_d.stride(0)
        if adj_d is not None:
            a.adjust_ids, a.adjust_vals = adj_d[0].data_ptr(), adj_d[1].data_ptr()
            a.adjust_row_stride, a.adjust_width = adj_d[0].stride(0), adj_d[0].shape[1]
            a.adjust_lens = adj_d[2].data_ptr()
        a.stream = stream.cuda_stream
        argv.append(a)
    lib_mod.check(L.vws_sample(ctypes.byref(argv[0])))
    torch.cuda.synchronize()
    n = parity_rows
    gflags = flags.cpu().numpy().view(np.uint32)
    prm = O.make_params(n, w.temperature[:n], w.top_k[:n], w.top_p[:n], w.min_p[:n],
                        w.repetition[:n], w.presence[:n], w.frequency[:n])
    ref = O.sample(w.logits_f32()[:n], prm, w.uniforms[:n],
                   output_ids=None if out_ids is None else out_ids[:n],
                   num_logprobs=num_logprobs, allowed=None if words is None else words[:n],
                   adjust_ids=None if adjust is None else adjust[0][:n],
                   adjust_vals=None if adjust is None else adjust[1][:n])
    mism = int((out.cpu().numpy()[:n] != ref["token"]).sum())
    if lp is not None:
        mism += int((lp[1].cpu().numpy()[:n] != ref["lp_ids"]).any(axis=1).sum())
        mism += int((lp[3].cpu().numpy()[:n] != ref["ranks"]).sum())
    for i in range(warmup):
        lib_mod.check(L.vws_sample(ctypes.byref(argv[i % len(argv)])))
    t = timed_region(lambda i: L.vws_sample(ctypes.byref(argv[i % len(argv)])), steps, stream)
    return {"kernel_us": kernel_us(t), "timing": t, "parity_rows": n, "mismatches": mism,
            "general_path_rows": int(((gflags & 0x100) != 0).sum())}


def cpu_baseline(w, rows: int, iters: int):
    """torch CPU restatement of vLLM's sampler on `rows` rows of the workload, all host cores."""
    import torch

    from oracle import vllm_torch as VT

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    sl = slice(0, rows)
    args = dict(temperature=torch.from_numpy(w.temperature[sl]), top_k=torch.from_numpy(w.top_k[sl]),
                top_p=torch.from_numpy(w.top_p[sl]), min_p=torch.from_numpy(w.min_p[sl]),
                repetition=torch.from_numpy(w.repetition[sl]), presence=torch.from_numpy(w.presence[sl]),
                frequency=torch.from_numpy(w.frequency[sl]),
                uniforms=torch.from_numpy(w.uniforms[sl]),
                output_ids=torch.from_numpy(w.output_ids[sl]))
    x = torch.from_numpy(w.logits_f32()[sl])
    for _ in range(3):
        VT.sample(x, **args)
    times = []
    for _ in range(iters):
        t0 = time.perf_counter_ns()
        VT.sample(x, **args)
        times.append((time.perf_counter_ns() - t0) * 1e-9)
    med = float(np.median(times))
    return dict(value=rows / med, unit="rows/s", cores=cores, kind="port",
                sample=(f"{rows} rows of C3 (V=128256, same seeded inputs), oracle/vllm_torch.py "
                        f"(vLLM-v1 Sampler op sequence on torch CPU tensors), median of {iters} "
                        f"after 3 warm-up, torch threads={cores}"),
                seconds_per_iter=med)


def cpu_reference_ops(w, rows: int, iters: int):
    """The reference's own host arithmetic, restated in numpy, timed on `rows` rows of the
    workload: greedy ``logits.argmax(axis=-1)`` over the batch (vllm_webgpu/v1/model_runner.py:145)
    and the CLI's float64 temperature sampler per row (run_inference.py:386-390: x / T - max, exp,
    normalise, ``np.random.choice``).  Single-threaded numpy, as the reference runs them."""
    x = w.logits_f32()[:rows]
    T = float(w.temperature[0]) if float(w.temperature[0]) > 0 else 1.0
    rng = np.random.RandomState(0)

    def greedy():
        return x.argmax(axis=-1)

    def cli_sampler():
        out = np.empty(x.shape[0], np.int64)
        for b in range(x.shape[0]):
            z = x[b].astype(np.float64) / T
            z = np.exp(z - z.max())
            out[b] = rng.choice(z.shape[0], p=z / z.sum())
        return out

    res = []
    for name, fn, cite in (("numpy greedy argmax", greedy, "vllm_webgpu/v1/model_runner.py:145"),
                           ("numpy float64 temperature sampler", cli_sampler,
                            "run_inference.py:386-390")):
        fn()
        times = []
        for _ in range(iters):
            t0 = time.perf_counter_ns()
            fn()
            times.append((time.perf_counter_ns() - t0) * 1e-9)
        med = float(np.median(times))
        res.append(dict(value=rows / med, unit="rows/s", cores=1, kind="port", op=name,
                        sample=f"{rows} rows of {w.name} (V={w.shape[1]}), median of {iters}, "
                               f"restates {cite}"))
    return res


PROFILE_SUMMARIES = {1: "sample_c1_b1_v32000.md", 2: "sample_c2_b64_v32000.md",
                     3: "sample_c3_b256_v128256.md", 4: "sample_c4_b512_v262144_bf16.md",
                     5: "sample_c5_b1024_v151936.md"}


def pmc_traffic_bytes(config: int):
    """HBM bytes per row_kernel launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    (copy-calibrated); None when no summary covers this workload."""
    name = PROFILE_SUMMARIES.get(config)
    if name is None:
        return None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"^\| `void vws::row_kernel<[a-z0-9 ,]+>\([^`]*` \|(?:[^|\n]*\|){5} *([0-9.]+) *\|$",
                  text, re.M)
    return None if m is None else float(m.group(1)) * 1e6


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--sets", type=int, default=3, help="rotated input sets (MALL defeat)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=256)
    ap.add_argument("--cpu-iters", type=int, default=30)
    ap.add_argument("--skip-v1", action="store_true",
                    help="skip the v1 Sampler.forward and generated-uniform timings (profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 512 MiB device copy (for PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU: the sampler shards by rows and "
                          "runs no collectives; run with --gpus 1"}), flush=True)
        sys.exit(2)

    import torch

    from vllm_webgpu_amd import _lib, ops
    from vllm_webgpu_amd import workloads as W

    t_gen = time.time()
    w = W.config(args.config)
    B, V = w.shape
    log(f"workload {w.name} B={B} V={V} generated in {time.time() - t_gen:.1f}s")
    dev = torch.device("cuda:0")
    L = _lib.lib()

    if w.dtype == "bf16":
        logits0 = torch.from_numpy(w.logits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        logits0 = torch.from_numpy(w.logits).to(dev)
    U0 = torch.from_numpy(w.uniforms).to(dev) if w.uniforms is not None else None
    H0 = torch.from_numpy(w.output_ids).to(dev) if w.output_ids is not None else None
    T = torch.from_numpy(w.temperature).to(dev)
    K = torch.from_numpy(w.top_k).to(dev)
    P = torch.from_numpy(w.top_p).to(dev)
    MP = torch.from_numpy(w.min_p).to(dev)
    R = torch.from_numpy(w.repetition).to(dev)
    PR = torch.from_numpy(w.presence).to(dev)
    FR = torch.from_numpy(w.frequency).to(dev)
    sets = []
    for i in range(args.sets):
        lg = torch.roll(logits0, shifts=i, dims=0).contiguous()
        u = torch.roll(U0, shifts=i, dims=0).contiguous() if U0 is not None else None
        h = torch.roll(H0, shifts=i, dims=0).contiguous() if H0 is not None else None
        sets.append((lg, u, h))
    out = torch.empty(B, dtype=torch.int32, device=dev)
    flags = torch.empty(B, dtype=torch.int32, device=dev)
    nkept = torch.empty(B, dtype=torch.int32, device=dev)
    ws = ops.workspace(L.vws_sample_workspace_size(B, V, 0 if H0 is None else H0.shape[1]), dev)
    lp = None
    if w.num_logprobs is not None:
        nl = w.num_logprobs
        lp = (nl, torch.empty((B, nl + 1), dtype=torch.int32, device=dev),
              torch.empty((B, nl + 1), dtype=torch.float32, device=dev),
              torch.empty(B, dtype=torch.int32, device=dev))
    stream = torch.cuda.current_stream()
    argv = []
    for lg, u, h in sets:
        a = build_args(_lib, lg, T, K, P, MP, R, PR, FR, h, u, out, flags, nkept, ws, lp)
        a.stream = stream.cuda_stream
        argv.append(a)
    sample = L.vws_sample

    # correctness spot check of set 0 against the oracle (tokens bit-exact)
    _lib.check(sample(ctypes.byref(argv[0])))
    torch.cuda.synchronize()
    gpu_tok = out.cpu().numpy()
    gpu_kept = nkept.cpu().numpy()
    gpu_flags = flags.cpu().numpy().view(np.uint32)
    from oracle import sampler as O  # checker only

    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence, w.frequency)
    ref = O.sample(w.logits_f32(), prm, w.uniforms, output_ids=w.output_ids,
                   num_logprobs=w.num_logprobs)
    mism = int((ref["token"] != gpu_tok).sum())
    parity = {"rows": int(B), "token_mismatches": mism,
              "flag_mismatches": int(((ref["flags"] & 0xFF) != (gpu_flags & 0xFF)).sum()),
              "kept_mismatches": int((ref["n_kept"] != gpu_kept).sum()),
              "checker": "oracle/vws_oracle.c on the same inputs (set 0)"}
    near_tie = {"top_p": int(((gpu_flags & 1) != 0).sum()), "race": int(((gpu_flags & 2) != 0).sum())}
    if w.return_probs:
        # C1 also returns the temperature-1 probabilities (vws_softmax)
        probs, rmax, _ = ops.softmax(sets[0][0], torch.ones(B))
        torch.cuda.synchronize()
        rp, rrm, _ = O.softmax(w.logits_f32(), 1.0)
        rel = np.abs(probs.cpu().numpy() - rp) / np.maximum(rp, 1e-30)
        parity["probs_max_rel_err"] = float(rel[rp > 1e-30].max())
        parity["row_max_mismatches"] = int((rmax.cpu().numpy() != rrm).sum())
    log(f"parity vs oracle: {parity}; |S| mean {gpu_kept.mean():.1f}; near-tie rows {near_tie}")
    if mism or parity["flag_mismatches"] or parity["kept_mismatches"]:
        print(json.dumps({"error": f"parity failure: {parity}"}), flush=True)
        sys.exit(1)

    # one step: vws_sample over the batch; C1 also returns its softmax probabilities
    probs_out = None
    if w.return_probs:
        probs_out = torch.empty((B, V), dtype=torch.float32, device=dev)
        pmax = torch.empty(B, dtype=torch.float32, device=dev)
        plsum = torch.empty(B, dtype=torch.float32, device=dev)
        ones = torch.ones(B, dtype=torch.float32, device=dev)
        softmax = L.vws_softmax

        def step(i):
            lg = sets[i % len(sets)][0]
            sample(ctypes.byref(argv[i % len(argv)]))
            softmax(lg.data_ptr(), _lib.DTYPE_F32, B, V, lg.stride(0), ones.data_ptr(),
                    probs_out.data_ptr(), pmax.data_ptr(), plsum.data_ptr(), stream.cuda_stream)
    else:
        def step(i):
            sample(ctypes.byref(argv[i % len(argv)]))

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # timed region: exactly `steps` calls, bracketed by synchronisation (wall clock: ms/step and
    # the rows/s value) and by two hipEvents on the launch stream (region time, dispatch gaps
    # included).  Then the same `steps` calls once more with every launch carrying an event
    # pair that the runtime stamps when the kernel itself begins and ends (hipExtLaunchKernel,
    # on the launch stream): their mean is the sampling kernel's average launch duration, the
    # figure a rocprofv3 kernel trace reports, from which the roofline is computed.
    nls = 2 if w.return_probs else 1
    tr = timed_region(step, args.steps, stream, nls, kernel_events=False)
    tk = timed_region(step, args.steps, stream, nls, kernel_events=True)
    st = L.vws_last_error()
    if st:
        log(f"last error: {st}")
    ms_per_step = tr["wall_s"] * 1e3 / args.steps
    rows_per_s = B * args.steps / tr["wall_s"]
    kern_us = kernel_us(tk)
    kern_ms = kern_us * 1e-3 if probs_out is None else (kern_us + kernel_us(tk, "softmax")) * 1e-3
    region_us = tr["region_ms"] / args.steps * 1e3

    alg_bytes = W.algorithmic_bytes(w, gpu_kept)
    gbps_e2e = alg_bytes / (ms_per_step * 1e-3) / 1e9
    gbps_kern = alg_bytes / (kern_ms * 1e-3) / 1e9
    log(f"ms/step {ms_per_step:.4f}  sampling kernel {kern_us:.2f} us (region {region_us:.2f} us "
        f"per step)  alg bytes {alg_bytes}  e2e {gbps_e2e:.0f} GB/s ({gbps_e2e / PEAK_HBM_GBPS:.1%})"
        f"  kernel {gbps_kern:.0f} GB/s ({gbps_kern / PEAK_HBM_GBPS:.1%})  raw {tr} {tk}")

    # the same step through the vLLM-v1 front end (Sampler.forward on a SamplingMetadata), with
    # the uniforms generated in the kernel from one key per row (no [B, V] tensor), and the
    # kernel alone in that mode
    # the same launch without the history (the penalty step skipped): what re-hashing the
    # padded histories every step costs inside the launch
    nohist = None
    if H0 is not None and not args.skip_v1:
        nohist = history_free_timing(_lib, L, sets, T, K, P, MP, R, PR, FR, out, flags, nkept,
                                     ws, lp, stream, min(args.steps, 300), min(args.warmup, 30))
        log(f"the same launch without the history: {kernel_us(nohist):.2f} us  raw {nohist}")
    tstate = None
    if H0 is not None and not args.skip_v1:
        tstate = token_state_timing(_lib, L, W, w, sets, T, K, P, MP, R, PR, FR, out, flags, nkept,
                                    ws, lp, stream, min(args.steps, 300), min(args.warmup, 30))
        log("token-state table: " + ", ".join(
            f"{k} {v['kernel_us']:.2f} us ({v['token_mismatches']} of {v['parity_rows']} rows "
            f"differ, {v['general_path_rows']} on the multi-pass path)" for k, v in tstate.items()))
    variants = None
    vsteps, vwarm = min(args.steps, 300), min(args.warmup, 30)
    if args.config == 3 and not args.skip_v1:
        one_masked = np.ones((B, V), bool)   # row 0 restricted to 20 tokens, the rest allowed
        one_masked[0] = False
        one_masked[0, np.random.default_rng(62).choice(V, 20, replace=False)] = True
        variants = {
            "logprobs_20": variant_timing(_lib, L, w, sets, T, K, P, MP, R, PR, FR, out, flags,
                                          nkept, ws, stream, vsteps, vwarm, num_logprobs=20),
            "one_masked_row": variant_timing(_lib, L, w, sets, T, K, P, MP, R, PR, FR, out, flags,
                                             nkept, ws, stream, vsteps, vwarm, allowed=one_masked)}
    elif args.config == 5 and not args.skip_v1:
        # C5 with C3's penalties (a 512-token output history per row; repetition 1.1,
        # presence 0.5, frequency 0.3)
        hist5 = np.random.default_rng(W.SEED_BASE + 35).integers(0, V, (B, 512), dtype=np.int64).astype(np.int32)
        w.repetition[:], w.presence[:], w.frequency[:] = 1.1, 0.5, 0.3
        R.fill_(1.1)
        PR.fill_(0.5)
        FR.fill_(0.3)
        ws5 = ops.workspace(L.vws_sample_workspace_size(B, V, 512), dev)
        variants = {
            # the history as the runner keeps it: the token-state table and its bitmap
            "c3_penalties_table": variant_timing(_lib, L, w, sets, T, K, P, MP, R, PR, FR, out,
                                                 flags, nkept, ws5, stream, vsteps, vwarm,
                                                 num_logprobs=w.num_logprobs, hist=hist5,
                                                 table=True),
            # the same history as padded id lists (the multi-pass path serves such rows)
            "c3_penalties": variant_timing(_lib, L, w, sets, T, K, P, MP, R, PR, FR, out,
                                           flags, nkept, ws5, stream, vsteps, vwarm,
                                           num_logprobs=w.num_logprobs, hist=hist5)}
        w.repetition[:], w.presence[:], w.frequency[:] = 1.0, 0.0, 0.0
        R.fill_(1.0)
        PR.fill_(0.0)
        FR.fill_(0.0)
        # C5 without logprobs, and the same with one row restricted to 20 tokens (an allowed
        # mask for the whole launch, all-ones on the other rows)
        one_masked5 = np.ones((B, V), bool)
        one_masked5[3] = False
        one_masked5[3, np.random.default_rng(68).choice(V, 20, replace=False)] = True
        variants["no_logprobs"] = variant_timing(_lib, L, w, sets, T, K, P, MP, R, PR, FR, out,
                                                 flags, nkept, ws, stream, vsteps, vwarm)
        variants["no_logprobs_one_masked_row"] = variant_timing(
            _lib, L, w, sets, T, K, P, MP, R, PR, FR, out, flags, nkept, ws, stream, vsteps,
            vwarm, allowed=one_masked5)
        # one row with a processor list (four banned ids: a min-tokens request), lengths given
        # so that the other rows carry none: that row takes the multi-pass path
        ids5 = np.full((B, 8), V, np.int32)
        vals5 = np.zeros((B, 8), np.float32)
        lens5 = np.zeros(B, np.int32)
        ids5[3, :4] = [11, 222, 3333, 44444]
        vals5[3, :4] = -np.inf
        lens5[3] = 4
        ws5b = ops.workspace(L.vws_sample_workspace_size(B, V, 8), dev)
        variants["one_row_with_bans"] = variant_timing(
            _lib, L, w, sets, T, K, P, MP, R, PR, FR, out, flags, nkept, ws5b, stream, vsteps,
            vwarm, num_logprobs=w.num_logprobs, adjust=(ids5, vals5, lens5))
    if variants:
        log("variants: " + ", ".join(
            f"{k} {v['kernel_us']:.2f} us ({v['mismatches']} mismatches in {v['parity_rows']} rows, "
            f"{v['general_path_rows']} rows on the multi-pass path)" for k, v in variants.items()))
    v1 = gen = None
    if not args.skip_v1:
        v1 = v1_forward_timing(w, sets[0][0], T, K, P, MP, R, PR, FR, sets[0][2], dev,
                               min(args.steps, 300), min(args.warmup, 30))
        gen = generated_timing(_lib, L, sets, T, K, P, MP, R, PR, FR, out, flags, nkept, ws,
                               lp, stream, B, min(args.steps, 300), min(args.warmup, 30))
        log(f"v1 Sampler.forward: {v1['wall_us']:.1f} us/step wall, {v1['gpu_us']:.1f} us/step on "
            f"the stream; kernel with generated uniforms "
            f"{kernel_us(gen):.2f} us  raw {gen}")

    if args.calibrate_copy:
        a = torch.empty(1 << 27, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        a.fill_(1.0)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        log("calibration copy: 536870912 bytes read + 536870912 bytes written")

    cpu = None
    cpu_ref_ops = None
    if not args.no_cpu_baseline:
        t = time.time()
        cpu = cpu_baseline(w, min(args.cpu_rows, B), args.cpu_iters)
        log(f"cpu baseline {cpu['value']:.1f} rows/s on {cpu['cores']} cores ({time.time() - t:.1f}s)")
        t = time.time()
        cpu_ref_ops = cpu_reference_ops(w, min(32, B), 5)
        log(f"reference numpy ops: {[round(c['value'], 1) for c in cpu_ref_ops]} rows/s "
            f"({time.time() - t:.1f}s)")

    res = {
        "metric": METRIC if args.config == 3 else f"sampled rows/sec + HBM GB/s (% peak), {w.name}",
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == "bf16" else "f32",
        "data": "synthetic",
        "config": {
            "workload": ("C3: fp32 logits B=256 V=128256 ~N(0,3); 512-token output history "
                         "(repetition 1.1, presence 0.5, frequency 0.3); T=0.7, top-k 50, "
                         "top-p 0.9; caller uniforms [B,V]; 3 rotated input sets")
            if args.config == 3 else f"{w.name}; {args.sets} rotated input sets",
            "global_batch": B, "vocab": V, "parallelism": "none (1 GPU)",
        },
        "hbm_gbps_end_to_end": gbps_e2e,
        "hbm_frac_end_to_end": gbps_e2e / PEAK_HBM_GBPS,
        "algorithmic_bytes_per_step": alg_bytes,
        "mean_survivors": float(gpu_kept.mean()),
        "parity": parity,
        "near_tie_rows": near_tie,
        "kernel_us": {"sample" if probs_out is None else "sample+softmax": kern_ms * 1e3},
        "region_us_per_step": region_us,
        # raw figures of every timed region: hipEvent-bracketed region ms, wall seconds, and per
        # kernel kind the summed kernel-stamped ms and the number of launches they cover
        "timing": tr,
        "timing_kernel_events": tk,
        "kernel_us_generated_uniforms": None if gen is None else kernel_us(gen),
        "timing_generated_uniforms": gen,
        "kernel_us_without_history": None if nohist is None else kernel_us(nohist),
        "timing_without_history": nohist,
        "kernel_us_long_history": (None if tstate is None
                                   else tstate["long_history_4096_1024"]["kernel_us"]),
        "token_state": tstate,
        "variants": variants,
        "v1_sampler_forward": None if v1 is None else {
            **v1, "kernel_us": kern_ms * 1e3, "wall_vs_kernel": v1["wall_us"] / (kern_ms * 1e3)},
        "roofline": {
            "bound": "hbm", "achieved": gbps_kern, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": gbps_kern / PEAK_HBM_GBPS, "traffic": pmc_traffic_bytes(args.config),
            # the instantiation the launch ran: element type, raw logprobs, logit transform
            # (0: none; the bench's workloads have no allowed mask and no soft cap)
            "kernel": "vws::row_kernel<{}, {}, 0>".format(
                "unsigned short" if w.dtype == "bf16" else "float",
                "true" if w.num_logprobs is not None else "false"),
        },
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "cpu_baseline_reference_ops": cpu_ref_ops,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()

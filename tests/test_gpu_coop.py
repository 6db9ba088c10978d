"""GPU parity of the cooperative passes: top-p rows whose finish needs another pass over their
logits (exact masses, wide race, rank) split it into chunks that other workgroups of the launch
run, through the fixed region at the start of the workspace.

Every total a chunk adds is an integer sum or an order-independent race merge, so the rows must
match the oracle bit for bit whoever ran which chunk.  The batches mix many wide rows with
short top-k rows (whose workgroups end early and help), in both dispatch modes: every row with
a workgroup of its own (B <= the workgroups the device holds at once) and more rows than that
(the launch counts its workgroups and starts the top-p rows first).  After each launch the
region must be ready for the next one: every slot free with no chunk open, the workgroup
counters at zero."""
import numpy as np
import pytest

from tests.cases import _wl
from tests.common import assert_same, gpu_run, oracle_run

pytestmark = pytest.mark.gpu

WIDE = 0x800
RECOUNT = 0x400

# CoopState layout (vllm_webgpu_amd/csrc/vws_internal.h): wgs (u64) at 0, then 16 slots of
# 34408 bytes from byte 256; a slot's claim word (u64) at +0, done (u32) at +32, owner at +36.
SLOTS, SLOT0, SLOT_BYTES = 16, 256, 34408


def _mixed(B, V, n_wide, seed):
    """n_wide wide top-p rows (flat logits, T 1.4, p 0.995) spread over a batch of top-k rows."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    wide = np.zeros(B, bool)
    wide[rng.choice(B, n_wide, replace=False)] = True
    x[wide] = rng.normal(0, 1.5, (n_wide, V)).astype(np.float32)
    T = np.where(wide, 1.4, 0.8).astype(np.float32)
    k = np.where(wide, 0, 50).astype(np.int32)
    p = np.where(wide, 0.995, 0.9).astype(np.float32)
    return _wl(f"coop B{B}", x, T, k=k, p=p, seed=seed), wide


def _region_clean(device):
    import torch

    from vllm_webgpu_amd import ops

    torch.cuda.synchronize()
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = ops._ws_cache[idx]
    head = ws[: SLOT0 + SLOTS * SLOT_BYTES].cpu().numpy()
    wgs = int(head[:8].view(np.uint64)[0])
    assert wgs == 0, f"workgroup counters left at {wgs:#x}"
    for s in range(SLOTS):
        base = SLOT0 + s * SLOT_BYTES
        claim = int(head[base:base + 8].view(np.uint64)[0])
        owner = int(head[base + 36:base + 40].view(np.uint32)[0])
        assert owner == 0, f"slot {s} still held by row {owner - 1}"
        assert (claim >> 32) & 0xFF == 0, f"slot {s} left with chunks open ({claim:#x})"


@pytest.mark.parametrize("B,V,n_wide", [(48, 65536, 24), (320, 65536, 40)])
def test_wide_rows_share_their_passes(cuda, B, V, n_wide):
    w, wide = _mixed(B, V, n_wide, seed=60 + B)
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), w.name)
    # most of the flat rows need the exact pass and the wide race (4 chunks of 4096 vectors
    # at this V, so they are shared)
    assert int(((g["flags"][wide] & WIDE) != 0).sum()) >= n_wide // 2
    _region_clean(cuda)


def test_back_to_back_launches_and_a_shared_workspace(cuda):
    """The region left by one launch serves the next, also after the top-k operation used the
    same workspace (its layout keeps the region and lays its own counters after it)."""
    import torch

    from vllm_webgpu_amd import ops

    w, _ = _mixed(300, 65536, 30, seed=71)
    ref = oracle_run(w)
    for _ in range(3):
        assert_same(gpu_run(w, cuda), ref, w.name)
    _region_clean(cuda)
    x = torch.from_numpy(w.logits).to(cuda)
    vals, ids = ops.topk(x, 100)
    torch.cuda.synchronize()
    assert_same(gpu_run(w, cuda), ref, w.name + " after topk")
    _region_clean(cuda)


def test_wide_rows_with_logprobs_and_bf16(cuda):
    """Wide rows with raw logprobs (the rank pass may run too) and bf16 logits."""
    w, wide = _mixed(280, 65536, 24, seed=73)
    w.num_logprobs = 5
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), w.name + " L=5")
    xb = w.logits_f32()
    u = xb.view(np.uint32).astype(np.uint64)
    w.logits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    w.dtype = "bf16"
    w.num_logprobs = None
    g = gpu_run(w, cuda)
    assert_same(g, oracle_run(w), w.name + " bf16")
    assert int(((g["flags"][wide] & (WIDE | RECOUNT)) != 0).sum()) >= w.shape[0] // 40
    _region_clean(cuda)


@pytest.mark.parametrize("B", [48, 320])
def test_given_up_passes_fall_back_and_free_their_slots(cuda, B):
    """With the owners' wait set to 0 polls from the host, every row that opens a shared pass
    gives it up once its own chunks are done and hands itself to the multi-pass path (reason 9
    in bits 16-23); the slot is freed by the owner when no other workgroup still runs a chunk
    of it, else by the last such chunk.  Every kernel still ends normally; every row must match
    the oracle, and the region must be clean after each launch and serve the next one at the
    default bound."""
    from vllm_webgpu_amd import _lib

    L = _lib.lib()
    w, wide = _mixed(B, 65536, 24, seed=81 + B)
    ref = oracle_run(w)
    gave_up = 0
    prev = L.vws_set_coop_wait_polls(0)
    try:
        for i in range(3):
            g = gpu_run(w, cuda)
            assert_same(g, ref, f"{w.name} polls=0 launch {i}")
            _region_clean(cuda)
            gave_up += int((((g["flags"] >> 16) & 0xFF) == 9).sum())
    finally:
        L.vws_set_coop_wait_polls(prev)
    print(f"B={B}: {gave_up} rows gave up a shared pass over 3 launches", flush=True)
    assert gave_up > 0
    g = gpu_run(w, cuda)
    assert_same(g, ref, w.name + " default bound")
    _region_clean(cuda)

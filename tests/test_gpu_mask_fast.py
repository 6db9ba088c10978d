"""GPU parity of allowed-token masks on the single passes: a launch with an allowed mask and no
logprobs masks every element as it streams -- one mask word per lane and iteration, shared
across the wave -- so its top-k, greedy and top-p rows no longer take the multi-pass path; a
launch with an allowed mask and raw logprobs streams raw values and masks the candidates of its
top-k and greedy rows.

Tokens, flags and survivor counts are compared bit for bit with the oracle."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import _wl
from tests.common import assert_same
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu

GENERAL = 0x100


def _bits(allowed):
    """bool [B, V] -> uint32 [B, ceil(V/32)] words (bit t & 31 of word t >> 5)."""
    B, V = allowed.shape
    words = np.zeros((B, (V + 31) // 32 * 32), np.uint64)
    words[:, :V] = allowed
    return (words.reshape(B, -1, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)


def _run(w, allowed, device, logits_t=None, num_logprobs=None, softcap=None, **kw):
    import torch

    from vllm_webgpu_amd import ops

    bits = _bits(allowed)
    prm = O.make_params(w.shape[0], w.temperature, w.top_k, w.top_p, w.min_p, w.repetition,
                        w.presence, w.frequency)
    ref = O.sample(w.logits_f32(), prm, w.uniforms, output_ids=w.output_ids, allowed=bits,
                   num_logprobs=num_logprobs, softcap=softcap, **{k: v for k, v in kw.items()})
    if logits_t is None:
        if w.dtype == "bf16":
            logits_t = torch.from_numpy(w.logits.view(np.int16)).to(device).view(torch.bfloat16)
        else:
            logits_t = torch.from_numpy(w.logits).to(device)
    greedy_all = bool(np.all(~(w.temperature >= np.float32(1e-5))))
    tk = {k: torch.from_numpy(v) for k, v in kw.items()}
    res = ops.sample(
        logits_t, temperature=None if greedy_all else torch.from_numpy(w.temperature),
        top_k=torch.from_numpy(w.top_k), top_p=torch.from_numpy(w.top_p),
        min_p=torch.from_numpy(w.min_p), repetition_penalty=torch.from_numpy(w.repetition),
        presence_penalty=torch.from_numpy(w.presence),
        frequency_penalty=torch.from_numpy(w.frequency),
        output_ids=None if w.output_ids is None else torch.from_numpy(w.output_ids),
        uniforms=torch.from_numpy(w.uniforms).to(device),
        allowed_mask=torch.from_numpy(bits.view(np.int32)).to(device), num_logprobs=num_logprobs,
        logit_softcap=softcap, **tk)
    torch.cuda.synchronize()
    g = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
             n_kept=res.num_kept.cpu().numpy())
    if num_logprobs is not None:
        g.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                 ranks=res.logprob_ranks.cpu().numpy())
    return g, ref


def _allowed_sets(rng, B, V):
    """Per row: 1 token, 5 tokens, 50, 1000, half the vocabulary, everything, nothing but the
    row's lowest logits region, in turn."""
    allowed = np.zeros((B, V), bool)
    for b in range(B):
        kind = b % 7
        if kind == 5:
            allowed[b] = True
        elif kind == 4:
            allowed[b] = rng.random(V) < 0.5
        else:
            n = (1, 5, 50, 1000, 0, 0, 300)[kind]
            allowed[b, rng.choice(V, n, replace=False)] = True
    return allowed


def test_c3_full_shape_with_masks(cuda):
    """C3 (256 x 128256 fp32, penalties from 512-token histories, T 0.7, top-k 50, top-p 0.9)
    with an allowed mask on every row: every row stays on the single pass."""
    w = W.config(3)
    rng = np.random.default_rng(61)
    allowed = _allowed_sets(rng, 256, 128256)
    g, ref = _run(w, allowed, cuda)
    assert_same(g, ref, "C3 + masks")
    n = int(((g["flags"] & GENERAL) != 0).sum())
    assert n == 0, f"{n} of 256 rows took the multi-pass path"


def test_c3_one_masked_row(cuda):
    """The bench's variant: C3 with one row restricted (the others allow everything)."""
    w = W.config(3)
    allowed = np.ones((256, 128256), bool)
    allowed[0] = False
    allowed[0, np.random.default_rng(62).choice(128256, 20, replace=False)] = True
    g, ref = _run(w, allowed, cuda)
    assert_same(g, ref, "C3 one masked row")
    assert not (g["flags"] & GENERAL).any()


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_16bit_logits_odd_vocab_and_greedy(cuda, dt):
    """8 elements per 16-byte vector, an odd vocabulary (a masked tail element by element),
    greedy rows and k above 64."""
    rng = np.random.default_rng(63)
    B, V = 56, 70001
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    T = np.where(np.arange(B) % 5 == 0, 0.0, 0.9).astype(np.float32)
    k = np.array([20, 50, 100, 1, 256, 7, 64] * 8, np.int32)
    w = _wl(f"{dt} masks", x, T, k=k, p=0.9, seed=64)
    if dt == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        w.logits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    else:
        w.logits = x.astype(np.float16)
    w.dtype = dt
    allowed = _allowed_sets(rng, B, V)
    allowed[:, V - 1] = rng.random(B) < 0.5   # the tail element itself masked or not
    g, ref = _run(w, allowed, cuda)
    assert_same(g, ref, w.name)


def test_unaligned_rows_and_processors(cuda):
    """Rows that start unaligned (a row stride of V + 1 elements: those rows take the
    multi-pass path) and masks together with penalties, bans and a positive bias (the
    up-front processed values see the mask too)."""
    import torch

    rng = np.random.default_rng(65)
    B, V = 24, 40000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    hist = rng.integers(0, V, (B, 200)).astype(np.int32)
    w = _wl("unaligned + processors", x, 0.8, k=30, p=0.9, rep=1.2, pres=0.3, freq=0.1,
            hist=hist, seed=66)
    allowed = _allowed_sets(rng, B, V)
    aid = rng.integers(0, V, (B, 8)).astype(np.int32)
    aval = np.where(rng.random((B, 8)) < 0.4, -np.inf, rng.normal(0, 4, (B, 8))).astype(np.float32)
    aval[:, 0] = 8.0  # a positive bias: the up-front path
    big = torch.zeros((B, V + 1), dtype=torch.float32, device=cuda)
    big[:, :V] = torch.from_numpy(x).to(cuda)
    g, ref = _run(w, allowed, cuda, logits_t=big[:, :V], adjust_ids=aid, adjust_vals=aval)
    assert_same(g, ref, w.name)
    g2, ref2 = _run(w, allowed, cuda, adjust_ids=aid, adjust_vals=aval)
    assert_same(g2, ref2, w.name + " aligned")


STREAM_TOPP = 0x200


def test_c5_topp_rows_with_masks(cuda):
    """C5's top-p rows (1024 x 151936 fp32, T 1, top-p 0.95, no top-k; without logprobs) with an
    allowed mask on every row -- one token, 5, 50, 1000, half the vocabulary, everything, 300:
    the top-p stream masks as it loads, so the rows stay on it."""
    w = W.config(5)
    w.num_logprobs = None
    B, V = w.shape
    rng = np.random.default_rng(67)
    allowed = _allowed_sets(rng, B, V)
    g, ref = _run(w, allowed, cuda)
    assert_same(g, ref, "C5 + masks")
    on = (g["flags"] & STREAM_TOPP) != 0
    assert on.mean() > 0.95, f"{int((~on).sum())} of {B} rows left the top-p stream"


def test_c5_one_masked_row(cuda):
    """The bench's variant: C5 (no logprobs) with one row restricted to 20 tokens."""
    w = W.config(5)
    w.num_logprobs = None
    B, V = w.shape
    allowed = np.ones((B, V), bool)
    allowed[3] = False
    allowed[3, np.random.default_rng(68).choice(V, 20, replace=False)] = True
    g, ref = _run(w, allowed, cuda)
    assert_same(g, ref, "C5 one masked row")
    # (the further passes some rows need mask their logits too)
    assert (g["flags"] & STREAM_TOPP).all()


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_topp_masks_small_rows_flat_rows_and_tails(cuda, dt):
    """Top-p rows with masks at every density, T != 1, min-p, greedy rows, flat rows whose
    nucleus reaches below the candidates (further passes over the masked logits, shared with
    other workgroups), an odd vocabulary (the tail element by element), and a row with nothing
    allowed."""
    rng = np.random.default_rng(69)
    B, V = 42, 60001
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[::6] = rng.normal(0, 0.3, (7, V)).astype(np.float32)  # flat rows
    T = np.where(np.arange(B) % 7 == 3, 0.0, np.where(np.arange(B) % 2 == 0, 1.0, 0.8)).astype(np.float32)
    mp = np.where(np.arange(B) % 5 == 1, 0.05, 0.0).astype(np.float32)
    w = _wl(f"{dt} top-p masks", x, T, k=0, p=0.92, mp=mp, seed=70)
    if dt == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        w.logits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    elif dt == "f16":
        w.logits = x.astype(np.float16)
    w.dtype = dt
    allowed = _allowed_sets(rng, B, V)
    allowed[:, V - 1] = rng.random(B) < 0.5
    allowed[41] = False
    g, ref = _run(w, allowed, cuda)
    assert_same(g, ref, w.name)


def test_topp_masks_flat_rows_take_the_passes(cuda):
    """Flat rows with half their vocabulary allowed: the nucleus reaches below the candidates,
    so the exact recount and the wide race run over the masked logits, in chunks shared with
    other workgroups; a few steeper rows in the same launch."""
    rng = np.random.default_rng(73)
    B, V = 40, 120000
    x = rng.normal(0, 0.4, (B, V)).astype(np.float32)
    x[::5] *= 8.0
    w = _wl("flat + masks", x, 0.9, k=0, p=0.97, seed=74)
    allowed = rng.random((B, V)) < 0.5
    g, ref = _run(w, allowed, cuda)
    assert_same(g, ref, w.name)
    assert (g["flags"] & STREAM_TOPP).all()
    assert (g["flags"] & (0x400 | 0x800)).any(), "no masked row took a further pass"


@pytest.mark.parametrize("case", ["c3_L20", "c4_bf16_L5"])
def test_logprob_launches_with_masks(cuda, case):
    """Raw logprobs and an allowed mask in one launch: the top-k and greedy rows mask their
    candidates on the single pass (the logprobs are of the raw logits); rows whose masked
    candidates reach the top k, and top-p rows, take the multi-pass path.  C3 (penalties,
    k 50, 20 logprobs) and a quarter of C4 (bf16, mixed rows, 5 logprobs), with masks of every
    density and half the rows left open; then the same launch with the single pass switched
    off (vws_set_single_pass), every top-k row on the multi-pass path, with the same results."""
    from vllm_webgpu_amd import _lib

    rng = np.random.default_rng(171)
    if case == "c3_L20":
        w, L = W.config(3), 20
    else:
        w, L = W.config(4, scale=0.25), 5
    B, V = w.shape
    allowed = _allowed_sets(rng, B, V)
    allowed[rng.random(B) < 0.5] = True                      # half the rows left open
    g, ref = _run(w, allowed, cuda, num_logprobs=L)
    assert_same(g, ref, case)
    open_rows = allowed.all(axis=1) & (w.top_k > 0) & (w.top_k <= 256)
    assert open_rows.sum() > 10
    gen = (g["flags"][open_rows] & GENERAL) != 0
    assert not gen.any(), f"{int(gen.sum())} open top-k rows took the multi-pass path"
    lib = _lib.lib()
    prev = lib.vws_set_single_pass(0)
    try:
        g2, _ = _run(w, allowed, cuda, num_logprobs=L)
    finally:
        lib.vws_set_single_pass(prev)
    assert_same(g2, ref, case + ", single pass off")
    assert ((g2["flags"][w.top_k > 0] & GENERAL) != 0).all()

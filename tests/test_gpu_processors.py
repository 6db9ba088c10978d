"""GPU parity of the logits processors (allowed-token mask, bans, logit bias) against the oracle:
the single-pass path (bans and negative biases found by raw value, positive biases gathered up
front), the multi-pass path (allowed masks, top-k off, logprobs), with and without penalties,
fp32 and bf16.  Token ids, flags and survivor counts must be bit-exact."""
import numpy as np
import pytest
import torch

from oracle import sampler as O
from tests.common import FLAG_MASK
from vllm_webgpu_amd import ops
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu


def _bits(allowed):
    B, V = allowed.shape
    Wd = (V + 31) // 32
    padded = np.zeros((B, Wd * 32), np.uint64)
    padded[:, :V] = allowed
    words = (padded.reshape(B, Wd, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2)
    return words.astype(np.uint32)


def _adjust(rng, x, width, ban_top=3, pos_bias=False, neg_bias=True):
    """Sparse processor lists: each row bans its ban_top largest logits plus random tokens, and
    biases random tokens (negative, or either sign with pos_bias)."""
    B, V = x.shape
    ids = np.full((B, width), V, np.int32)          # padding
    vals = np.zeros((B, width), np.float32)
    for b in range(B):
        top = np.argsort(-x[b], kind="stable")[:ban_top]
        rest = rng.choice(V, size=width - ban_top, replace=False)
        rest = rest[~np.isin(rest, top)][: width - ban_top]
        ids[b, :ban_top] = top
        vals[b, :ban_top] = -np.inf
        n = rest.size
        ids[b, ban_top:ban_top + n] = rest
        lo, hi = (-4.0, 4.0) if pos_bias else (-4.0, -0.5)
        v = rng.uniform(lo, hi, n).astype(np.float32)
        v[rng.random(n) < 0.25] = -np.inf
        if not neg_bias:
            v = np.abs(v)
        vals[b, ban_top:ban_top + n] = v
    return ids, vals


def _run(cuda, w, logits_np, ids=None, vals=None, allowed=None, L=None, softcap=None):
    B, V = w.shape
    if w.dtype == "bf16":
        lg = torch.from_numpy(w.logits.view(np.int16)).to(cuda).view(torch.bfloat16)
    else:
        lg = torch.from_numpy(logits_np).to(cuda)
    greedy_all = bool(np.all(~(w.temperature >= np.float32(1e-5))))
    U = torch.from_numpy(w.uniforms).to(cuda) if w.uniforms is not None else None
    res = ops.sample(
        lg, temperature=None if greedy_all else torch.from_numpy(w.temperature),
        top_k=torch.from_numpy(w.top_k), top_p=torch.from_numpy(w.top_p),
        min_p=torch.from_numpy(w.min_p), repetition_penalty=torch.from_numpy(w.repetition),
        presence_penalty=torch.from_numpy(w.presence), frequency_penalty=torch.from_numpy(w.frequency),
        output_ids=None if w.output_ids is None else torch.from_numpy(w.output_ids), uniforms=U,
        num_logprobs=L,
        allowed_mask=None if allowed is None else torch.from_numpy(_bits(allowed).view(np.int32)).to(cuda),
        adjust_ids=None if ids is None else torch.from_numpy(ids),
        adjust_vals=None if vals is None else torch.from_numpy(vals), logit_softcap=softcap)
    torch.cuda.synchronize()
    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                        w.frequency)
    ref = O.sample(w.logits_f32(), prm, w.uniforms, output_ids=w.output_ids, num_logprobs=L,
                   allowed=None if allowed is None else _bits(allowed), adjust_ids=ids,
                   adjust_vals=vals, softcap=softcap)
    tok = res.sampled.cpu().numpy()
    fl = res.flags.cpu().numpy().view(np.uint32)
    bad = np.nonzero(tok != ref["token"])[0]
    assert bad.size == 0, f"rows {bad[:8]}: gpu {tok[bad[:8]]} oracle {ref['token'][bad[:8]]} flags {fl[bad[:8]]}"
    np.testing.assert_array_equal(fl & FLAG_MASK, ref["flags"] & FLAG_MASK)
    np.testing.assert_array_equal(res.num_kept.cpu().numpy(), ref["n_kept"])
    if L is not None:
        np.testing.assert_array_equal(res.logprob_ids.cpu().numpy(), ref["lp_ids"])
        np.testing.assert_allclose(res.logprob_vals.cpu().numpy(), ref["lp_vals"], rtol=1e-5, atol=1e-6)
    return tok, fl


@pytest.mark.parametrize("pos_bias", [False, True])
def test_single_pass_rows_with_bans_and_bias(cuda, pos_bias):
    w = W.config(3, scale=0.05)                   # top-k 50 rows with penalties
    rng = np.random.default_rng(5 + pos_bias)
    x = w.logits_f32()
    ids, vals = _adjust(rng, x, 40, ban_top=3, pos_bias=pos_bias)
    tok, fl = _run(cuda, w, w.logits, ids, vals)
    top = np.argsort(-x, axis=1)[:, :3]
    assert not np.any(tok[:, None] == top)         # the three banned maxima never come out
    assert not np.any(fl & 0x100)                  # served by the single-pass path


def test_greedy_rows_with_processors(cuda):
    w = W.config(4, scale=0.05)                    # bf16, 1/8 greedy rows, mixed parameters
    rng = np.random.default_rng(9)
    ids, vals = _adjust(rng, w.logits_f32(), 24, ban_top=2, pos_bias=True)
    _run(cuda, w, None, ids, vals)


def test_multi_pass_rows_with_mask_and_logprobs(cuda):
    w = W.config(5, scale=0.05)                    # top-p only, logprobs
    B, V = w.shape
    rng = np.random.default_rng(13)
    allowed = rng.random((B, V)) < 0.5
    allowed[:, 0] = True
    ids, vals = _adjust(rng, w.logits_f32(), 32, ban_top=2, pos_bias=True)
    tok, fl = _run(cuda, w, w.logits, ids, vals, allowed=allowed, L=w.num_logprobs)
    assert np.all(allowed[np.arange(B), tok])


def test_mask_on_top_k_rows(cuda):
    w = W.config(2, scale=0.25)                    # top-k rows mask on the single pass
    B, V = w.shape
    rng = np.random.default_rng(17)
    allowed = rng.random((B, V)) < 0.1
    allowed[:, 1] = True
    tok, fl = _run(cuda, w, w.logits, allowed=allowed)
    assert np.all(allowed[np.arange(B), tok]) and not np.any(fl & 0x100)


def test_long_processor_lists(cuda):
    w = W.config(3, scale=0.05)
    B, V = w.shape
    rng = np.random.default_rng(21)
    width = 1300                                   # more entries than threads per row
    ids = np.stack([rng.choice(V, width, replace=False) for _ in range(B)]).astype(np.int32)
    vals = rng.uniform(-3.0, -0.1, (B, width)).astype(np.float32)
    vals[:, ::7] = -np.inf
    _run(cuda, w, w.logits, ids, vals)


def test_processor_lengths_keep_other_rows_on_their_paths(cuda):
    """With per-row lengths, only the rows that carry processor entries leave the top-p path
    (the others of a launch with a list are not counted as carrying one); parity throughout."""
    rng = np.random.default_rng(131)
    B, V = 32, 50000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    ids = np.full((B, 6), V, np.int32)
    vals = np.zeros((B, 6), np.float32)
    lens = np.zeros(B, np.int32)
    for b in (3, 17):
        ids[b, :4] = np.argsort(-x[b])[:4]     # ban the row's four largest logits
        vals[b, :4] = -np.inf
        lens[b] = 4
    T = np.full(B, 0.9, np.float32)
    p = np.full(B, 0.92, np.float32)
    u = rng.random((B, V), dtype=np.float32).clip(2 ** -24, 1 - 2 ** -24)
    prm = O.make_params(B, T, np.zeros(B, np.int32), p, np.zeros(B, np.float32),
                        np.ones(B, np.float32), np.zeros(B, np.float32), np.zeros(B, np.float32))
    ref = O.sample(x, prm, u, adjust_ids=ids, adjust_vals=vals, adjust_lens=lens)
    res = ops.sample(torch.from_numpy(x).to(cuda), temperature=torch.from_numpy(T),
                     top_p=torch.from_numpy(p), uniforms=torch.from_numpy(u).to(cuda),
                     adjust_ids=torch.from_numpy(ids), adjust_vals=torch.from_numpy(vals),
                     adjust_lens=torch.from_numpy(lens))
    torch.cuda.synchronize()
    tok = res.sampled.cpu().numpy()
    fl = res.flags.cpu().numpy().view(np.uint32)
    assert np.array_equal(tok, ref["token"])
    assert np.array_equal(fl & FLAG_MASK, ref["flags"] & FLAG_MASK)
    general = (fl & 0x100) != 0
    assert general[[3, 17]].all() and general.sum() == 2

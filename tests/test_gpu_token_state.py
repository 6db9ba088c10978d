"""GPU parity of the per-request token-state table: the penalties' history given as
one uint32 word per (request, token) -- prompt flag in bit 31, output count below -- instead of
padded prompt/output id lists.

The table is built here from the same id lists with numpy (np.add.at / bitwise_or.at, an
encoding independent of the library), the GPU samples with the table, and the oracle samples
with the lists: token ids, flags and survivor counts must match bit for bit.  Long histories
(4096-token prompts plus 1024-token outputs, more distinct ids than the single pass's LDS hash
holds) must stay on the single pass with the table; the table's maintenance kernel must
reproduce the numpy table exactly."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import _wl
from tests.common import assert_same

pytestmark = pytest.mark.gpu

GENERAL = 0x100
PROMPT = np.uint32(0x80000000)


def table_from_lists(B, V, prompt=None, output=None, plens=None, olens=None):
    """uint32 [B, V]: prompt flag | output count, from padded id lists (ids outside [0, V) and
    columns past the lengths are padding)."""
    st = np.zeros((B, V), np.uint32)
    for ids, lens, is_prompt in ((prompt, plens, True), (output, olens, False)):
        if ids is None:
            continue
        W = ids.shape[1]
        cols = np.arange(W)[None, :]
        ok = (ids >= 0) & (ids < V)
        if lens is not None:
            ok &= cols < lens[:, None]
        rows = np.broadcast_to(np.arange(B)[:, None], ids.shape)[ok]
        t = ids[ok].astype(np.int64)
        if is_prompt:
            np.bitwise_or.at(st, (rows, t), PROMPT)
        else:
            np.add.at(st, (rows, t), np.uint32(1))
    return st


def _dev_table(st, device):
    import torch

    return torch.from_numpy(st.view(np.int32)).to(device)


def _oracle(w, prompt=None, output=None, plens=None, olens=None, **kw):
    B = w.shape[0]
    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                        w.frequency)
    return O.sample(w.logits_f32(), prm, w.uniforms, prompt_ids=prompt, output_ids=output,
                    prompt_lens=plens, output_lens=olens, num_logprobs=w.num_logprobs, **kw)


def _gpu(w, device, token_state=None, token_state_rows=None, prompt=None, output=None, **kw):
    import torch

    from vllm_webgpu_amd import ops

    x = torch.from_numpy(w.logits).to(device)
    greedy_all = bool(np.all(~(w.temperature >= np.float32(1e-5))))
    res = ops.sample(
        x, temperature=None if greedy_all else torch.from_numpy(w.temperature),
        top_k=torch.from_numpy(w.top_k), top_p=torch.from_numpy(w.top_p),
        min_p=torch.from_numpy(w.min_p), repetition_penalty=torch.from_numpy(w.repetition),
        presence_penalty=torch.from_numpy(w.presence),
        frequency_penalty=torch.from_numpy(w.frequency),
        prompt_ids=None if prompt is None else torch.from_numpy(prompt),
        output_ids=None if output is None else torch.from_numpy(output),
        uniforms=torch.from_numpy(w.uniforms).to(device), num_logprobs=w.num_logprobs,
        token_state=token_state, token_state_rows=token_state_rows, **kw)
    torch.cuda.synchronize()
    out = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
               n_kept=res.num_kept.cpu().numpy())
    if w.num_logprobs is not None:
        out.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                   ranks=res.logprob_ranks.cpu().numpy())
    return out


def _long_history(B, V, n_prompt, n_out, rep, pres, freq, seed, k=50, p=0.9, T=0.7):
    """C3-like rows whose histories hit the rows' top tokens: each row's 40 largest logits are
    planted into its prompt and output (the latter 1-4 times), the rest drawn uniformly."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    prompt = rng.integers(0, V, (B, n_prompt), dtype=np.int64).astype(np.int32)
    out = rng.integers(0, V, (B, n_out), dtype=np.int64).astype(np.int32)
    top = np.argsort(-x, axis=1)[:, :40].astype(np.int32)
    prompt[:, :20] = top[:, ::2]
    reps = np.repeat(top[:, 1::2], 4, axis=1)[:, : min(80, n_out)]
    out[:, : reps.shape[1]] = reps
    w = _wl(f"long history B{B} V{V} {n_prompt}+{n_out}", x, T, k=k, p=p, rep=rep, pres=pres,
            freq=freq, seed=seed)
    return w, prompt, out


@pytest.mark.parametrize("rep,pres,freq", [(1.1, 0.5, 0.3), (1.0, 0.5, 0.3), (1.3, 0.0, 0.0)])
def test_long_history_full_c3_shape_stays_on_the_single_pass(cuda, rep, pres, freq):
    """C3's shape (256 x 128256 fp32, T 0.7, top-k 50, top-p 0.9) with a 4096-token prompt and
    a 1024-token output per row: with the table, every row is served by the single pass and
    matches the oracle run on the id lists."""
    w, prompt, out = _long_history(256, 128256, 4096, 1024, rep, pres, freq, seed=901)
    ref = _oracle(w, prompt=prompt, output=out)
    st = table_from_lists(256, 128256, prompt, out)
    g = _gpu(w, cuda, token_state=_dev_table(st, cuda))
    assert_same(g, ref, w.name + " table")
    assert not (g["flags"] & GENERAL).any(), f"{int(((g['flags'] & GENERAL) != 0).sum())} rows left the single pass"


def test_long_history_lists_still_match(cuda):
    """The same long histories as id lists: rows whose distinct ids overflow the LDS hash take
    the multi-pass path and still match; at repetition 1 the prompt ids are not hashed, so the
    1024-token outputs alone stay on the single pass."""
    w, prompt, out = _long_history(64, 128256, 4096, 1024, 1.1, 0.5, 0.3, seed=902)
    g = _gpu(w, cuda, prompt=prompt, output=out)
    assert_same(g, _oracle(w, prompt=prompt, output=out), w.name + " lists")
    w1, prompt1, out1 = _long_history(64, 128256, 4096, 1024, 1.0, 0.5, 0.3, seed=903)
    g1 = _gpu(w1, cuda, prompt=prompt1, output=out1)
    assert_same(g1, _oracle(w1, prompt=prompt1, output=out1), w1.name + " lists rep 1")
    assert not (g1["flags"] & GENERAL).any()


def test_table_rows_map_and_short_histories(cuda):
    """A table whose rows are stored in another order (token_state_rows), with extra unused
    rows, padded/short histories, greedy rows mixed in: same results as the lists."""
    import torch

    B, V = 96, 50000
    w, prompt, out = _long_history(B, V, 300, 200, 1.2, 0.4, 0.2, seed=904)
    rng = np.random.default_rng(5)
    plens = rng.integers(0, 301, B).astype(np.int32)
    olens = rng.integers(0, 201, B).astype(np.int32)
    w.temperature[::7] = 0.0  # greedy rows: argmax of the penalised logits
    ref = _oracle(w, prompt=prompt, output=out, plens=plens, olens=olens)
    st = table_from_lists(B, V, prompt, out, plens, olens)
    perm = rng.permutation(B + 13)[:B].astype(np.int32)  # table row of each batch row
    big = np.zeros((B + 13, V + 64), np.uint32)           # wider rows than V, unused rows
    big[perm, :V] = st
    big[np.setdiff1d(np.arange(B + 13), perm), :V] = 7    # garbage in rows nobody reads
    g = _gpu(w, cuda, token_state=_dev_table(big, cuda),
             token_state_rows=torch.from_numpy(perm))
    assert_same(g, ref, "table with a row map")


@pytest.mark.parametrize("case", ["raising", "topp_only", "bias", "logprobs", "minp"])
def test_table_on_the_other_paths(cuda, case):
    """Rows the single pass hands on: penalties that may raise a logit (r < 1, negative
    presence), top-p without top-k, processors with a positive bias, a launch with logprobs,
    min-p; all with the table, against the oracle on the lists."""
    import torch

    B, V = 48, 40000
    kw = {}
    if case == "raising":
        w, prompt, out = _long_history(B, V, 500, 300, 0.8, -0.5, 0.1, seed=911)
    elif case == "topp_only":
        w, prompt, out = _long_history(B, V, 500, 300, 1.1, 0.5, 0.3, seed=912, k=0, p=0.8)
    elif case == "logprobs":
        w, prompt, out = _long_history(B, V, 500, 300, 1.1, 0.5, 0.3, seed=913)
        w.num_logprobs = 5
    elif case == "minp":
        w, prompt, out = _long_history(B, V, 500, 300, 1.1, 0.5, 0.3, seed=914, k=200, p=0.95)
        w.min_p[:] = 0.05
    else:
        w, prompt, out = _long_history(B, V, 500, 300, 1.1, 0.5, 0.3, seed=915)
        rng = np.random.default_rng(16)
        aid = rng.integers(0, V, (B, 6)).astype(np.int32)
        aval = np.where(rng.random((B, 6)) < 0.3, -np.inf, rng.normal(0, 3, (B, 6))).astype(np.float32)
        aid[:, 0] = np.argsort(-w.logits, axis=1)[:, 60]   # a biased token near the top
        aval[:, 0] = 6.0
        kw = dict(adjust_ids=aid, adjust_vals=aval)
    ref = _oracle(w, prompt=prompt, output=out, **kw)
    st = table_from_lists(B, V, prompt, out)
    tk = {k: torch.from_numpy(v) for k, v in kw.items()}
    g = _gpu(w, cuda, token_state=_dev_table(st, cuda), **tk)
    assert_same(g, ref, f"table {case}")


def test_table_maintenance_matches_numpy(cuda):
    """vws_token_state_update: prompt flags per request (one row per call), then output ids
    appended step by step for a batch of rows (repeats included), equal the numpy table; ids
    outside [0, V) and negative rows are skipped."""
    import torch

    from vllm_webgpu_amd import ops

    R, V = 20, 3000
    rng = np.random.default_rng(21)
    state = torch.zeros((R, V + 5), dtype=torch.int32, device=cuda)
    prompts = [rng.integers(-2, V + 2, rng.integers(0, 400)).astype(np.int32) for _ in range(R)]
    for r, p in enumerate(prompts):
        ops.token_state_update(state, torch.from_numpy(p).to(cuda), rows=r, prompt=True, vocab=V)
    outs = np.full((R, 0), -1, np.int32)
    for _ in range(30):
        rows = rng.permutation(R)[:15].astype(np.int32)
        rows[3] = -1                                   # skipped
        tok = rng.integers(-1, V + 1, 15).astype(np.int32)
        tok[:4] = tok[4]                               # repeats within a call
        ops.token_state_update(state, torch.from_numpy(tok).to(cuda),
                               rows=torch.from_numpy(rows).to(cuda), vocab=V)
        col = np.full((R, 1), -1, np.int32)            # rows are distinct within a call
        col[rows[rows >= 0], 0] = tok[rows >= 0]
        outs = np.concatenate([outs, col], axis=1)
    torch.cuda.synchronize()
    W = max(len(p) for p in prompts)
    pad = np.full((R, W), -1, np.int32)
    for r, p in enumerate(prompts):
        pad[r, :len(p)] = p
    want = table_from_lists(R, V, pad, outs)
    got = state.cpu().numpy().view(np.uint32)
    assert np.array_equal(got[:, :V], want)
    assert not got[:, V:].any()

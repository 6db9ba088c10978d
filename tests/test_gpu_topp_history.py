"""GPU parity of top-p rows with penalties from the token-state table and its bitmap of non-zero
words: such rows stay on the single-pass top-p path, which stages the bitmap in LDS, buffers
every history token whatever its value and gives those tokens their processed values from their
words (the further passes over the row read the words of every element).

The table and bitmap are built with numpy from padded id lists (independently of the library),
the GPU samples with the table, the oracle with the lists: token ids, flags, survivor counts,
logprob ids and ranks bit for bit, logprob values within the tolerances of tests/common.py."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import _wl
from tests.common import assert_same
from tests.test_gpu_token_state import table_from_lists

pytestmark = pytest.mark.gpu

GENERAL = 0x100
STREAM_TOPP = 0x200
RECOUNT = 0x400
WIDE = 0x800


def bits_from_table(st):
    """int32 [R, ceil(V/32)]: bit t & 31 of word t >> 5 set where the table's word t is non-zero."""
    R, V = st.shape
    nz = np.zeros((R, (V + 31) // 32 * 32), np.uint64)
    nz[:, :V] = st != 0
    w = (nz.reshape(R, -1, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)
    return w.view(np.int32)


def _run(w, device, prompt=None, output=None, plens=None, olens=None, bits=True, softcap=None):
    import torch

    from vllm_webgpu_amd import ops

    B, V = w.shape
    prm = O.make_params(B, w.temperature, w.top_k, w.top_p, w.min_p, w.repetition, w.presence,
                        w.frequency)
    ref = O.sample(w.logits_f32(), prm, w.uniforms, prompt_ids=prompt, output_ids=output,
                   prompt_lens=plens, output_lens=olens, num_logprobs=w.num_logprobs,
                   softcap=softcap)
    st = table_from_lists(B, V, prompt, output, plens, olens)
    if w.dtype == "bf16":
        x = torch.from_numpy(w.logits.view(np.int16)).to(device).view(torch.bfloat16)
    else:
        x = torch.from_numpy(w.logits).to(device)
    greedy_all = bool(np.all(~(w.temperature >= np.float32(1e-5))))
    res = ops.sample(
        x, temperature=None if greedy_all else torch.from_numpy(w.temperature),
        top_k=torch.from_numpy(w.top_k), top_p=torch.from_numpy(w.top_p),
        min_p=torch.from_numpy(w.min_p), repetition_penalty=torch.from_numpy(w.repetition),
        presence_penalty=torch.from_numpy(w.presence),
        frequency_penalty=torch.from_numpy(w.frequency),
        uniforms=torch.from_numpy(w.uniforms).to(device), num_logprobs=w.num_logprobs,
        token_state=torch.from_numpy(st.view(np.int32)).to(device),
        token_state_bits=torch.from_numpy(bits_from_table(st)).to(device) if bits else None,
        logit_softcap=softcap)
    torch.cuda.synchronize()
    g = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
             n_kept=res.num_kept.cpu().numpy())
    if w.num_logprobs is not None:
        g.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                 ranks=res.logprob_ranks.cpu().numpy())
    return g, ref


def _hist(rng, x, n_prompt, n_out, top_share=40):
    """Histories that hit each row's largest logits: half of the top `top_share` ids in the
    prompt, the other half 1-4 times in the output, the rest uniform."""
    B, V = x.shape
    prompt = rng.integers(0, V, (B, n_prompt), dtype=np.int64).astype(np.int32)
    out = rng.integers(0, V, (B, n_out), dtype=np.int64).astype(np.int32)
    top = np.argsort(-x, axis=1)[:, :top_share].astype(np.int32)
    h = top_share // 2
    prompt[:, :min(h, n_prompt)] = top[:, ::2][:, :min(h, n_prompt)]
    reps = np.repeat(top[:, 1::2], 3, axis=1)[:, :n_out]
    out[:, :reps.shape[1]] = reps
    return prompt, out


def test_c5_with_c3_penalties_stays_on_the_topp_path(cuda):
    """C5's shape (1024 x 151936 fp32, T 1, top-p 0.95, 20 logprobs) with C3's penalties
    (repetition 1.1, presence 0.5, frequency 0.3) from a 512-token output history per row."""
    from vllm_webgpu_amd import workloads as W

    w = W.config(5)
    B, V = w.shape
    hist = np.random.default_rng(W.SEED_BASE + 35).integers(0, V, (B, 512), dtype=np.int64).astype(np.int32)
    w.repetition[:], w.presence[:], w.frequency[:] = 1.1, 0.5, 0.3
    g, ref = _run(w, cuda, output=hist)
    assert_same(g, ref, "C5 + penalties (table)")
    n = int(((g["flags"] & GENERAL) != 0).sum())
    assert n == 0, f"{n} of {B} rows took the multi-pass path"


@pytest.mark.parametrize("case", ["T07_L5", "T1_noL", "minp_L0", "raising", "greedy_L3", "long"])
def test_penalised_topp_rows(cuda, case):
    """Histories that penalise each row's top tokens, with and without raw logprobs, T != 1,
    min-p, penalties that raise logits (repetition < 1, negative presence), greedy rows asking
    for logprobs, and 4096 + 1024-token histories."""
    rng = np.random.default_rng({"T07_L5": 1, "T1_noL": 2, "minp_L0": 3, "raising": 4,
                                 "greedy_L3": 5, "long": 6}[case])
    B, V = 48, 60000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    n_prompt, n_out = (4096, 1024) if case == "long" else (300, 200)
    prompt, out = _hist(rng, x, n_prompt, n_out)
    kw = dict(rep=1.2, pres=0.4, freq=0.2)
    T, L, mp, p = 0.7, 5, 0.0, 0.9
    if case == "T1_noL":
        T, L = 1.0, None
    elif case == "minp_L0":
        mp, L, p = 0.02, 0, 0.95
    elif case == "raising":
        kw = dict(rep=0.8, pres=-0.5, freq=0.1)
    elif case == "greedy_L3":
        T, L = 0.0, 3
    w = _wl(case, x, T, k=0, p=p, mp=mp, seed=rng.integers(1 << 30), L=L, **kw)
    g, ref = _run(w, cuda, prompt=prompt, output=out)
    assert_same(g, ref, case)
    if case != "greedy_L3":   # greedy rows with logprobs: the single pass serves them
        assert (g["flags"] & STREAM_TOPP).all(), f"{case}: rows left the top-p path: {g['flags']}"


def test_flat_rows_take_the_passes_with_penalties(cuda):
    """Flat rows (the nucleus reaches below the candidates): the exact recount and the wide race
    pass apply the penalties from every element's word; the passes run in cooperation with
    other workgroups.  A few rows with steeper logits in the same launch."""
    rng = np.random.default_rng(71)
    B, V = 40, 120000
    x = rng.normal(0, 0.4, (B, V)).astype(np.float32)
    x[::5] *= 8.0
    prompt, out = _hist(rng, x, 500, 400, top_share=200)
    w = _wl("flat + penalties", x, 0.9, k=0, p=0.97, rep=1.3, pres=0.6, freq=0.3, seed=72, L=4)
    g, ref = _run(w, cuda, prompt=prompt, output=out)
    assert_same(g, ref, w.name)
    assert not (g["flags"] & GENERAL).any()
    assert (g["flags"] & (RECOUNT | WIDE)).any(), "no row took a further pass"


def test_capped_rows_with_penalties(cuda):
    """Under the soft cap (30): the stream caps as it loads, the history tokens' gathered logits
    are capped before their words apply, and flat rows take the capped passes; T 0.9, 3 raw
    logprobs, a few saturated rows."""
    rng = np.random.default_rng(111)
    B, V = 40, 90000
    x = rng.normal(0, 12, (B, V)).astype(np.float32)
    x[1::5] = rng.normal(0, 0.5, (8, V))
    x[::7, :30] = 500.0
    prompt, out = _hist(rng, x, 300, 200, top_share=60)
    w = _wl("cap + penalties", x, 0.9, k=0, p=0.95, rep=1.2, pres=0.4, freq=0.2, seed=112, L=3)
    g, ref = _run(w, cuda, prompt=prompt, output=out, softcap=30.0)
    assert_same(g, ref, w.name)
    assert ((g["flags"] & STREAM_TOPP) != 0).mean() > 0.9, f"rows left the top-p path: {g['flags']}"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_16bit_logits_and_unaligned_tails(cuda, dt):
    """8 elements per 16-byte vector, an odd vocabulary, history tokens in the unaligned tail."""
    rng = np.random.default_rng(81)
    B, V = 32, 50021
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    prompt, out = _hist(rng, x, 200, 150)
    out[:, -4:] = np.arange(V - 4, V, dtype=np.int32)  # the last tokens of the row
    w = _wl(f"{dt} + penalties", x, 0.8, k=0, p=0.9, rep=1.1, pres=0.3, freq=0.2, seed=82, L=2)
    if dt == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        w.logits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    else:
        w.logits = x.astype(np.float16)
    w.dtype = dt
    g, ref = _run(w, cuda, prompt=prompt, output=out)
    assert_same(g, ref, w.name)
    assert not (g["flags"] & GENERAL).any()


def test_without_bitmap_or_above_the_bitmap_vocab(cuda):
    """Without the bitmap, and with V above the LDS bitmap's 196608 tokens, the rows take the
    multi-pass path and still match."""
    rng = np.random.default_rng(91)
    x = rng.normal(0, 3, (8, 40000)).astype(np.float32)
    prompt, out = _hist(rng, x, 100, 100)
    w = _wl("no bitmap", x, 0.9, k=0, p=0.9, rep=1.2, pres=0.2, seed=92)
    g, ref = _run(w, cuda, prompt=prompt, output=out, bits=False)
    assert_same(g, ref, w.name)
    assert (g["flags"] & GENERAL).all()
    x = rng.normal(0, 3, (4, 200000)).astype(np.float32)
    prompt, out = _hist(rng, x, 100, 100)
    w = _wl("V 200000", x, 0.9, k=0, p=0.9, rep=1.2, pres=0.2, seed=93)
    g, ref = _run(w, cuda, prompt=prompt, output=out)
    assert_same(g, ref, w.name)
    assert (g["flags"] & GENERAL).all()


def test_bitmap_maintenance(cuda):
    """vws_token_state_update with the bitmap: the bits of every updated id are set, nothing
    else (prompt flags, then output ids, ids outside [0, V) and negative rows skipped)."""
    import torch

    from vllm_webgpu_amd import ops

    R, V = 12, 3000
    rng = np.random.default_rng(101)
    state = torch.zeros((R, V), dtype=torch.int32, device=cuda)
    bits = torch.zeros((R, (V + 31) // 32 + 3), dtype=torch.int32, device=cuda)
    for r in range(R):
        p = rng.integers(-2, V + 2, rng.integers(0, 300)).astype(np.int32)
        ops.token_state_update(state, torch.from_numpy(p).to(cuda), rows=r, prompt=True, bits=bits)
    for _ in range(20):
        rows = rng.permutation(R)[:8].astype(np.int32)
        rows[2] = -1
        tok = rng.integers(-1, V + 1, 8).astype(np.int32)
        ops.token_state_update(state, torch.from_numpy(tok).to(cuda),
                               rows=torch.from_numpy(rows).to(cuda), bits=bits)
    torch.cuda.synchronize()
    want = bits_from_table(state.cpu().numpy().view(np.uint32))
    got = bits.cpu().numpy()
    assert np.array_equal(got[:, :want.shape[1]], want)
    assert not got[:, want.shape[1]:].any()

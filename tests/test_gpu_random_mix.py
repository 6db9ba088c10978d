"""Randomised mixed launches against the oracle: every option the sampling call takes, combined
at random in one launch -- fp32, bf16 or f16 logits; greedy rows, top-k (1 to 300, off),
top-p, min-p; penalties from padded id lists or from the token-state table with its bitmap;
raw logprobs (0, 3 or 20); an allowed mask of random density per row; bans and biases with
per-row lengths; Gemma's soft cap with and without its f16 store; odd vocabularies.  Each
launch's rows take whichever paths their parameters pick (single pass, single-pass top-p with
its further passes, multi-pass), so the paths' hand-overs are exercised together.

Token ids, flags and survivor counts must match the oracle bit for bit; logprob ids and ranks
bit for bit, values within the tolerances of tests/common.py."""
import numpy as np
import pytest

from oracle import sampler as O
from tests.cases import _u
from tests.common import assert_same
from tests.test_gpu_topp_history import bits_from_table
from tests.test_gpu_token_state import table_from_lists

pytestmark = pytest.mark.gpu


def _words(allowed):
    B, V = allowed.shape
    w = np.zeros((B, (V + 31) // 32 * 32), np.uint64)
    w[:, :V] = allowed
    return (w.reshape(B, -1, 32) << np.arange(32, dtype=np.uint64)).sum(axis=2).astype(np.uint32)


def _launch(rng, dt, big=False):
    B = int(rng.integers(300, 700)) if big else int(rng.integers(8, 72))
    V = int(rng.choice([4099, 32000, 50021] if big else [4099, 32000, 50021, 128256, 151936]))
    x = rng.normal(0, rng.uniform(0.5, 5.0), (B, V)).astype(np.float32)
    x[rng.random(B) < 0.15] *= 0.05                                   # flat rows
    spikes = rng.integers(0, V, (B, 6))
    np.put_along_axis(x, spikes, x.max(axis=1, keepdims=True) + rng.uniform(0, 4, (B, 6)).astype(np.float32), 1)
    if rng.random() < 0.3:
        x = np.round(x * 4) / 4                                       # coarse grid: ties
    if dt == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        raw = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        xf = (raw.astype(np.uint32) << 16).view(np.float32)
    elif dt == "f16":
        raw = x.astype(np.float16)
        xf = raw.astype(np.float32)
    else:
        raw = xf = x
    T = np.where(rng.random(B) < 0.15, 0.0, rng.uniform(0.3, 1.5, B)).astype(np.float32)
    k = rng.choice(np.array([0, 0, 0, 1, 20, 50, 256, 300], np.int32), B).astype(np.int32)
    p = np.where(rng.random(B) < 0.3, 1.0, rng.uniform(0.5, 0.99, B)).astype(np.float32)
    mp = np.where(rng.random(B) < 0.2, 0.05, 0.0).astype(np.float32)
    cfg = dict(B=B, V=V, dt=dt, raw=raw, xf=xf, T=T, k=k, p=p, mp=mp,
               rep=np.ones(B, np.float32), pres=np.zeros(B, np.float32),
               freq=np.zeros(B, np.float32), prompt=None, output=None, table=False, L=None,
               allowed=None, aid=None, aval=None, alen=None, cap=None, cap16=False)
    if rng.random() < 0.6:
        cfg["rep"] = np.where(rng.random(B) < 0.7, rng.uniform(0.8, 1.3, B), 1.0).astype(np.float32)
        cfg["pres"] = np.where(rng.random(B) < 0.5, rng.uniform(-0.5, 0.8, B), 0.0).astype(np.float32)
        cfg["freq"] = np.where(rng.random(B) < 0.5, rng.uniform(0.0, 0.5, B), 0.0).astype(np.float32)
        W = int(rng.choice([16, 128, 512]))
        out = rng.integers(0, V, (B, W)).astype(np.int32)
        top = np.argsort(-xf, axis=1)[:, :8].astype(np.int32)         # hit the rows' top tokens
        out[:, :8] = top
        out[rng.random((B, W)) < 0.1] = V                             # padding
        cfg["output"] = out
        if rng.random() < 0.5:
            cfg["prompt"] = rng.integers(0, V, (B, 64)).astype(np.int32)
        cfg["table"] = rng.random() < 0.5
    cfg["L"] = [None, 0, 3, 20][int(rng.integers(0, 4))]
    if rng.random() < 0.3:
        dens = rng.choice([0.001, 0.1, 0.5, 1.0], B)
        allowed = rng.random((B, V)) < dens[:, None]
        allowed[np.arange(B), rng.integers(0, V, B)] = True
        cfg["allowed"] = allowed
    if rng.random() < 0.25:
        Wa = 6
        # distinct ids per row (at most one finite entry per token is the call's contract):
        # the row's top two, then four others
        top2 = np.argsort(-xf, axis=1)[:, :2]
        aid = np.empty((B, Wa), np.int32)
        for b in range(B):
            rest = rng.choice(V - 2, Wa - 2, replace=False)
            rest = np.setdiff1d(np.arange(V), top2[b])[rest]
            aid[b] = np.concatenate([top2[b], rest])
        aval = np.where(rng.random((B, Wa)) < 0.5, -np.inf, rng.uniform(-2, 2, (B, Wa))).astype(np.float32)
        cfg.update(aid=aid, aval=aval, alen=rng.integers(0, Wa + 1, B).astype(np.int32))
    if rng.random() < 0.25:
        cfg["cap"] = 30.0
        cfg["cap16"] = bool(rng.random() < 0.5)
    return cfg


@pytest.mark.parametrize("seed", range(60))
def test_random_mixed_launch(cuda, seed):
    """Seeds 48 and above use larger batches (up to 700 rows: more rows than workgroups resident
    at once) and the kernel's own uniforms (a launch-wide generator key)."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(5000 + seed)
    c = _launch(rng, ["f32", "bf16", "f16"][seed % 3], big=seed >= 48)
    B, V = c["B"], c["V"]
    key = int(rng.integers(1, 2 ** 62)) if seed >= 48 else None
    if key is None:
        u = _u(rng, (B, V))
    else:
        u = O.philox_uniforms(np.full(B, key, np.uint64), V, np.arange(B, dtype=np.uint64))
    prm = O.make_params(B, c["T"], c["k"], c["p"], c["mp"], c["rep"], c["pres"], c["freq"])
    bits = None if c["allowed"] is None else _words(c["allowed"])
    ref = O.sample(c["xf"], prm, u, prompt_ids=c["prompt"], output_ids=c["output"],
                   num_logprobs=c["L"], allowed=bits, adjust_ids=c["aid"],
                   adjust_vals=c["aval"], adjust_lens=c["alen"], softcap=c["cap"],
                   softcap_f16=c["cap16"])
    dev = cuda
    if c["dt"] == "bf16":
        x = torch.from_numpy(c["raw"].view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        x = torch.from_numpy(c["raw"]).to(dev)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    hist = {}
    if c["output"] is not None:
        if c["table"]:
            st = table_from_lists(B, V, c["prompt"], c["output"])
            hist = dict(token_state=t(st.view(np.int32)))
            if V <= 196608:
                hist["token_state_bits"] = t(bits_from_table(st))
        else:
            hist = dict(prompt_ids=t(c["prompt"]), output_ids=t(c["output"]))
    greedy_all = bool(np.all(~(c["T"] >= np.float32(1e-5))))
    res = ops.sample(
        x, temperature=None if greedy_all else torch.from_numpy(c["T"]),
        top_k=torch.from_numpy(c["k"]), top_p=torch.from_numpy(c["p"]),
        min_p=torch.from_numpy(c["mp"]), repetition_penalty=torch.from_numpy(c["rep"]),
        presence_penalty=torch.from_numpy(c["pres"]), frequency_penalty=torch.from_numpy(c["freq"]),
        uniforms=None if key is not None else t(u), rng_key=key, num_logprobs=c["L"],
        allowed_mask=None if bits is None else t(bits.view(np.int32)),
        adjust_ids=t(c["aid"]), adjust_vals=t(c["aval"]), adjust_lens=t(c["alen"]),
        logit_softcap=c["cap"], logit_softcap_f16=c["cap16"], **hist)
    torch.cuda.synchronize()
    g = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
             n_kept=res.num_kept.cpu().numpy())
    if c["L"] is not None:
        g.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                 ranks=res.logprob_ranks.cpu().numpy())
    label = (f"seed {seed}: {c['dt']} B={B} V={V} L={c['L']} pen={c['output'] is not None} "
             f"table={c['table']} mask={bits is not None} adj={c['aid'] is not None} cap={c['cap']}")
    print(label, flush=True)
    assert_same(g, ref, label)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_multi_pass_edges_are_not_duplicated(cuda, dt):
    """Multi-pass rows whose every element survives (no top-k, top-p 1), with the allowed mask
    masking the first and last tokens and penalties on them: the padding of the unaligned
    head, of the tail and of the chunks past the tail must not be processed into copies of
    those tokens (each would count as a survivor, and carry mass on top-p rows).  Odd
    vocabularies and a row view that starts unaligned, so that both edges are partial."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(77)
    B, V = 12, 4099
    x = rng.normal(0, 2, (B, V + 3)).astype(np.float32)
    T = np.full(B, 0.9, np.float32)
    k = np.zeros(B, np.int32)
    p = np.where(np.arange(B) % 3 == 2, 0.97, 1.0).astype(np.float32)
    rep = np.full(B, 1.2, np.float32)
    pres = np.full(B, 0.4, np.float32)
    out = np.tile(np.array([0, 1, 2, 3, 5, 7, V - 1, V - 2, V - 3], np.int32), (B, 1))
    allowed = rng.random((B, V)) < 0.5
    allowed[:, :8] = False
    allowed[:, V - 8:] = False
    allowed[:, 100] = True
    bits = _words(allowed)
    u = _u(rng, (B, V))
    for off in (0, 1):                                   # aligned rows, then rows off by one
        xv = x[:, off:off + V]
        if dt == "bf16":
            uu = np.ascontiguousarray(xv).view(np.uint32).astype(np.uint64)
            raw = ((uu + 0x7FFF + ((uu >> 16) & 1)) >> 16).astype(np.uint16)
            xf = (raw.astype(np.uint32) << 16).view(np.float32)
            full = torch.from_numpy(np.ascontiguousarray(
                np.pad(raw, ((0, 0), (off, 3 - off)))).view(np.int16)).to(cuda).view(torch.bfloat16)
        else:
            xf = np.ascontiguousarray(xv)
            full = torch.from_numpy(np.ascontiguousarray(np.pad(xf, ((0, 0), (off, 3 - off))))).to(cuda)
        xt = full[:, off:off + V]
        prm = O.make_params(B, T, k, p, 0.0, rep, pres, 0.0)
        ref = O.sample(xf, prm, u, output_ids=out, allowed=bits)
        res = ops.sample(xt, temperature=torch.from_numpy(T), top_k=torch.from_numpy(k),
                         top_p=torch.from_numpy(p), repetition_penalty=torch.from_numpy(rep),
                         presence_penalty=torch.from_numpy(pres),
                         output_ids=torch.from_numpy(out).to(cuda),
                         uniforms=torch.from_numpy(u).to(cuda),
                         allowed_mask=torch.from_numpy(bits.view(np.int32)).to(cuda))
        torch.cuda.synchronize()
        g = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
                 n_kept=res.num_kept.cpu().numpy())
        assert_same(g, ref, f"{dt} offset {off}")
        assert (g["n_kept"][p == 1.0] == V).all()


def _edge_launch(rng):
    """Extreme parameters: tiny and odd vocabularies, strided rows that start unaligned, NaN and
    infinite logits, extreme temperatures, k around V, p at 0 and near 1, min-p up to 1,
    histories with lengths (as lists, or as a token-state table reached through a row map),
    rows that allow nothing, bans and biases, the soft cap at 1 and 30."""
    B = int(rng.integers(1, 40))
    V = int(rng.choice([1, 2, 7, 63, 64, 65, 100, 1000, 3001, 8191, 8193, 20000]))
    off = int(rng.integers(0, 4))
    full = rng.normal(0, rng.choice([0.01, 1.0, 8.0]), (B, V + 4)).astype(np.float32)
    x = full[:, off:off + V]
    sp = rng.random((B, V))
    x = np.where(sp < 0.002, np.nan, x)
    x = np.where((sp >= 0.002) & (sp < 0.004), -np.inf, x)
    x = np.where((sp >= 0.004) & (sp < 0.0045), np.inf, x).astype(np.float32)
    if rng.random() < 0.3:
        x = np.round(x).astype(np.float32)                            # many ties
    T = rng.choice(np.array([0.0, 1e-3, 0.05, 1.0, 3.0, 10.0], np.float32), B).astype(np.float32)
    k = rng.choice(np.array([0, 1, 2, max(V - 1, 0), V, V + 5, 64, 65, 256, 257], np.int32), B).astype(np.int32)
    p = rng.choice(np.array([1.0, 0.999999, 0.5, 1e-6, 0.0, 0.3], np.float32), B).astype(np.float32)
    mp = rng.choice(np.array([0.0, 0.0, 0.5, 0.99, 1.0], np.float32), B).astype(np.float32)
    c = dict(B=B, V=V, off=off, x=x, T=T, k=k, p=p, mp=mp, rep=np.ones(B, np.float32),
             pres=np.zeros(B, np.float32), freq=np.zeros(B, np.float32), prompt=None,
             output=None, plens=None, olens=None, L=None, allowed=None, table=False,
             aid=None, aval=None, alen=None, cap=None, cap16=False)
    if rng.random() < 0.5:
        c["rep"] = rng.uniform(0.5, 2.0, B).astype(np.float32)
        c["pres"] = rng.uniform(-1.0, 1.0, B).astype(np.float32)
        c["freq"] = rng.uniform(-0.5, 0.5, B).astype(np.float32)
        W = int(rng.integers(1, 40))
        c["output"] = rng.integers(-2, V + 2, (B, W)).astype(np.int32)
        c["olens"] = rng.integers(0, W + 1, B).astype(np.int32)
        if rng.random() < 0.5:
            c["prompt"] = rng.integers(0, V, (B, W)).astype(np.int32)
            c["plens"] = rng.integers(0, W + 1, B).astype(np.int32)
    if rng.random() < 0.5:
        c["L"] = int(min(V, rng.choice([0, 1, 5, 20])))
    if rng.random() < 0.3:
        allowed = rng.random((B, V)) < rng.choice([0.0, 0.01, 0.5, 1.0], B)[:, None]
        c["allowed"] = allowed
    if c["output"] is not None and rng.random() < 0.5:
        c["table"] = True
    if rng.random() < 0.25:
        Wa = 4
        aid = np.full((B, Wa), -1, np.int32)
        for b in range(B):
            n = min(Wa, V)
            aid[b, :n] = rng.choice(V, n, replace=False)
        aval = np.where(rng.random((B, Wa)) < 0.4, -np.inf, rng.uniform(-3, 3, (B, Wa))).astype(np.float32)
        c.update(aid=aid, aval=aval, alen=rng.integers(0, Wa + 1, B).astype(np.int32))
    if rng.random() < 0.25:
        c["cap"] = float(rng.choice([1.0, 30.0]))
        c["cap16"] = bool(rng.random() < 0.5)
    return c


# 10285 and 10663: short history rows with 20 raw logprobs whose stream keeps every element,
# with a NaN history token (the top-p path listed it among the raw top L)
@pytest.mark.parametrize("seed", list(range(60)) + [10285, 10663])
def test_random_edge_launch(cuda, seed):
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(9000 + seed)
    c = _edge_launch(rng)
    B, V = c["B"], c["V"]
    u = _u(rng, (B, V))
    prm = O.make_params(B, c["T"], c["k"], c["p"], c["mp"], c["rep"], c["pres"], c["freq"])
    bits = None if c["allowed"] is None else _words(c["allowed"])
    ref = O.sample(c["x"], prm, u, prompt_ids=c["prompt"], output_ids=c["output"],
                   prompt_lens=c["plens"], output_lens=c["olens"], num_logprobs=c["L"],
                   allowed=bits, adjust_ids=c["aid"], adjust_vals=c["aval"],
                   adjust_lens=c["alen"], softcap=c["cap"], softcap_f16=c["cap16"])
    # the logits as a strided view of a wider buffer, starting c["off"] elements in
    buf = np.full((B, V + 4), np.float32(7.0))
    buf[:, c["off"]:c["off"] + V] = c["x"]
    xt = torch.from_numpy(buf).to(cuda)[:, c["off"]:c["off"] + V]
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    if c["table"]:
        # the histories as a token-state table of B + 3 rows, reached through a row map; the
        # rows no launch row maps to hold junk
        R = B + 3
        rows = rng.permutation(R)[:B].astype(np.int32)
        st = rng.integers(0, 2 ** 31, (R, V)).astype(np.uint32)
        st[rows] = table_from_lists(B, V, c["prompt"], c["output"], c["plens"], c["olens"])
        hist = dict(token_state=t(st.view(np.int32)), token_state_rows=t(rows))
        if V <= 196608:
            hist["token_state_bits"] = t(bits_from_table(st))
    else:
        hist = dict(prompt_ids=t(c["prompt"]), prompt_lens=t(c["plens"]),
                    output_ids=t(c["output"]), output_lens=t(c["olens"]))
    greedy_all = bool(np.all(~(c["T"] >= np.float32(1e-5))))
    res = ops.sample(
        xt, temperature=None if greedy_all else torch.from_numpy(c["T"]),
        top_k=torch.from_numpy(c["k"]), top_p=torch.from_numpy(c["p"]),
        min_p=torch.from_numpy(c["mp"]), repetition_penalty=torch.from_numpy(c["rep"]),
        presence_penalty=torch.from_numpy(c["pres"]), frequency_penalty=torch.from_numpy(c["freq"]),
        uniforms=t(u), num_logprobs=c["L"],
        allowed_mask=None if bits is None else t(bits.view(np.int32)),
        adjust_ids=t(c["aid"]), adjust_vals=t(c["aval"]), adjust_lens=t(c["alen"]),
        logit_softcap=c["cap"], logit_softcap_f16=c["cap16"], **hist)
    torch.cuda.synchronize()
    g = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
             n_kept=res.num_kept.cpu().numpy())
    if c["L"] is not None:
        g.update(lp_ids=res.logprob_ids.cpu().numpy(), lp_vals=res.logprob_vals.cpu().numpy(),
                 ranks=res.logprob_ranks.cpu().numpy())
    label = (f"edge seed {seed}: B={B} V={V} off={c['off']} L={c['L']} "
             f"pen={c['output'] is not None} table={c['table']} mask={bits is not None} "
             f"adj={c['aid'] is not None} cap={c['cap']}/{c['cap16']}")
    print(label, flush=True)
    assert_same(g, ref, label)


@pytest.mark.parametrize("seed", range(40))
def test_random_ops(cuda, seed):
    """The standalone operations on random edge inputs: argmax, top-k (k from 1 to min(V, 256)),
    softmax at a random temperature (fp32, bf16 or f16 logits), and the in-place penalties --
    tiny and odd vocabularies, NaN and infinite logits, heavy ties, strided rows."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(7000 + seed)
    B = int(rng.integers(1, 30))
    V = int(rng.choice([1, 2, 7, 64, 65, 1000, 4099, 32000, 40001]))
    x = rng.normal(0, rng.choice([0.01, 1.0, 8.0]), (B, V)).astype(np.float32)
    if rng.random() < 0.4:
        x = np.round(x * 2) / 2                                       # ties
    sp = rng.random((B, V))
    x = np.where(sp < 0.003, np.nan, x)
    x = np.where((sp >= 0.003) & (sp < 0.006), -np.inf, x)
    x = np.where((sp >= 0.006) & (sp < 0.007), np.inf, x).astype(np.float32)
    dt = ["f32", "bf16", "f16"][seed % 3]
    if dt == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        raw = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        xf = (raw.astype(np.uint32) << 16).view(np.float32)
        xt = torch.from_numpy(raw.view(np.int16)).to(cuda).view(torch.bfloat16)
    elif dt == "f16":
        raw = x.astype(np.float16)
        xf = raw.astype(np.float32)
        xt = torch.from_numpy(raw).to(cuda)
    else:
        xf = x
        wide = np.zeros((B, V + 3), np.float32)
        wide[:, 1:V + 1] = x
        xt = torch.from_numpy(wide).to(cuda)[:, 1:V + 1]            # strided, unaligned rows
    label = f"ops seed {seed}: {dt} B={B} V={V}"
    print(label, flush=True)

    assert np.array_equal(ops.argmax(xt).cpu().numpy(), O.argmax(xf)), label + " argmax"

    k = int(rng.integers(1, min(V, 256) + 1))
    vals, ids = ops.topk(xt, k)
    rv, ri = O.topk(xf, k)
    assert np.array_equal(ids.cpu().numpy(), ri), f"{label} topk ids (k={k})"
    # (values equal as floats: NaN to NaN, and -0 to +0, the keys the ordering uses)
    np.testing.assert_array_equal(vals.cpu().numpy(), rv, err_msg=f"{label} topk values")

    T = np.float32(rng.choice([0.05, 0.7, 1.0, 3.0]))
    p, rm, ls = ops.softmax(xt, torch.full((B,), float(T)))
    p, rm, ls = p.cpu().numpy(), rm.cpu().numpy(), ls.cpu().numpy()
    for b in range(B):
        rp, rrm, rls = O.softmax(xf[b:b + 1], float(T))
        np.testing.assert_allclose(p[b], rp[0], rtol=1e-5, atol=1e-12, equal_nan=True,
                                   err_msg=f"{label} softmax row {b}")
        assert rm[b] == rrm[0] or (np.isnan(rm[b]) and np.isnan(rrm[0])), f"{label} row max {b}"

    if dt == "f32":
        W = int(rng.integers(1, 30))
        pr = rng.integers(-1, V + 1, (B, W)).astype(np.int32)
        ou = rng.integers(-1, V + 1, (B, W)).astype(np.int32)
        rep = rng.uniform(0.5, 2.0, B).astype(np.float32)
        pres = rng.uniform(-1, 1, B).astype(np.float32)
        freq = rng.uniform(-1, 1, B).astype(np.float32)
        ref = O.apply_penalties(xf, pr, ou, rep, pres, freq)
        got = torch.from_numpy(xf.copy()).to(cuda)
        ops.apply_penalties(got, torch.from_numpy(rep), torch.from_numpy(pres),
                            torch.from_numpy(freq), prompt_ids=torch.from_numpy(pr).to(cuda),
                            output_ids=torch.from_numpy(ou).to(cuda))
        assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32)), label + " penalties"


@pytest.mark.parametrize("V,k", [(7, 6), (65, 64), (1000, 256)])
def test_banned_nan_logits(cuda, V, k):
    """A ban turns a NaN logit into -inf, which counts as a survivor when the top k reaches
    -inf (rows with fewer than k values that are not NaN), as the oracle's assignment does."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(V)
    B = 4
    x = rng.normal(0, 1, (B, V)).astype(np.float32)
    x[rng.random((B, V)) < 0.6] = np.nan
    aid = np.full((B, 3), -1, np.int32)
    aval = np.full((B, 3), -np.inf, np.float32)
    for b in range(B):
        nan_ids = np.flatnonzero(np.isnan(x[b]))
        aid[b, 0] = nan_ids[0]                          # a banned NaN
        aid[b, 1] = np.flatnonzero(~np.isnan(x[b]))[0]  # a banned value
        aid[b, 2] = nan_ids[-1]
        aval[b, 2] = 1.5                                 # a biased NaN stays NaN
    alen = np.array([3, 2, 1, 3], np.int32)
    T = np.array([1.0, 0.5, 0.0, 2.0], np.float32)
    kk = np.full(B, k, np.int32)
    p = np.ones(B, np.float32)
    zero, one = np.zeros(B, np.float32), np.ones(B, np.float32)
    u = _u(rng, (B, V))
    prm = O.make_params(B, T, kk, p, zero, one, zero, zero)
    ref = O.sample(x, prm, u, adjust_ids=aid, adjust_vals=aval, adjust_lens=alen)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    res = ops.sample(t(x), temperature=torch.from_numpy(T), top_k=torch.from_numpy(kk),
                     top_p=torch.from_numpy(p), uniforms=t(u), adjust_ids=t(aid),
                     adjust_vals=t(aval), adjust_lens=t(alen))
    torch.cuda.synchronize()
    g = dict(token=res.sampled.cpu().numpy(), flags=res.flags.cpu().numpy().view(np.uint32),
             n_kept=res.num_kept.cpu().numpy())
    assert_same(g, ref, f"banned NaN logits V={V} k={k}")

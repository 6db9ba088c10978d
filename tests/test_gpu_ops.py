"""GPU parity of the standalone penalty operation, and of operations sharing one workspace.

``vws_apply_penalties`` is the vLLM-v1 penalty step on its own (repetition on prompt and output
tokens, then frequency per occurrence, then presence), in place on fp32 logits.  The oracle's
``apply_penalties`` restates it.  Every operation of the library receives the same per-device
workspace from ``ops.workspace``; each must leave it as it found it, so a sequence
penalties -> top-k -> sample on one workspace must match the oracle op by op.
"""
import numpy as np
import pytest

from oracle import sampler as O
from tests.common import assert_same, gpu_run, oracle_run
from vllm_webgpu_amd import workloads as W

pytestmark = pytest.mark.gpu


def _hist(rng, B, H, V, pad_frac=0.2):
    """Padded int32 [B, H] histories with duplicates and padding ids (V, -1, V + 7)."""
    h = rng.integers(0, V, (B, H)).astype(np.int32)
    h[:, 1::7] = h[:, 0::7][:, : h[:, 1::7].shape[1]]        # duplicates
    pad = rng.random((B, H)) < pad_frac
    h[pad] = rng.choice(np.array([V, -1, V + 7], np.int32), size=int(pad.sum()))
    return h


@pytest.mark.parametrize("B,V,HP,HO", [(4, 1000, 40, 60), (16, 50257, 700, 1500), (3, 128256, 0, 512)])
def test_apply_penalties_parity(cuda, B, V, HP, HO):
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(B * 1000 + V)
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[:, :5] = np.array([0.0, -0.0, 2.5, -2.5, 1e-30], np.float32)  # signs at zero
    pr = _hist(rng, B, HP, V) if HP else None
    ou = _hist(rng, B, HO, V)
    ou[:, :3] = np.array([0, 1, 2], np.int32)
    rep = rng.uniform(0.8, 1.5, B).astype(np.float32)
    pres = rng.uniform(-0.5, 1.0, B).astype(np.float32)
    freq = rng.uniform(-0.2, 0.5, B).astype(np.float32)
    ref = O.apply_penalties(x, prompt_ids=pr, output_ids=ou, repetition=rep, presence=pres,
                            frequency=freq)
    t = torch.from_numpy(x).to(cuda)
    ops.apply_penalties(t, repetition_penalty=torch.from_numpy(rep),
                        presence_penalty=torch.from_numpy(pres),
                        frequency_penalty=torch.from_numpy(freq),
                        prompt_ids=None if pr is None else torch.from_numpy(pr),
                        output_ids=torch.from_numpy(ou))
    torch.cuda.synchronize()
    got = t.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert not np.array_equal(got, x)


def test_apply_penalties_lengths(cuda):
    """Per-row lengths cut the histories (entries past the length are ignored)."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(3)
    B, V, H = 5, 2048, 64
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    ou = rng.integers(0, V, (B, H)).astype(np.int32)
    lens = np.array([0, 1, 17, 63, 64], np.int32)
    cut = ou.copy()
    for b in range(B):
        cut[b, lens[b]:] = V
    ref = O.apply_penalties(x, output_ids=cut, repetition=1.3, presence=0.4, frequency=0.2)
    t = torch.from_numpy(x).to(cuda)
    ops.apply_penalties(t, repetition_penalty=1.3, presence_penalty=0.4, frequency_penalty=0.2,
                        output_ids=torch.from_numpy(ou), output_lens=torch.from_numpy(lens))
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_penalties_then_topk_then_sample_shared_workspace(cuda):
    """Regression: the penalty op once left its history hash in the shared workspace, where the
    top-k op keeps its per-row part counters; top-k rows then never elected a last part and
    returned uninitialised memory."""
    import torch

    from vllm_webgpu_amd import ops

    rng = np.random.default_rng(11)
    B, V, H = 12, 30011, 900
    x = np.round(rng.normal(size=(B, V)) * 8).astype(np.float32) / 8
    ou = rng.integers(0, V, (B, H)).astype(np.int32)
    for rnd in range(2):
        t = torch.from_numpy(x).to(cuda)
        ops.apply_penalties(t, repetition_penalty=1.2, presence_penalty=0.3, frequency_penalty=0.1,
                            output_ids=torch.from_numpy(ou))
        ref_pen = O.apply_penalties(x, output_ids=ou, repetition=1.2, presence=0.3, frequency=0.1)
        for k in (1, 50, 256):
            vals, ids = ops.topk(t, k)
            rv, ri = O.topk(ref_pen, k)
            assert np.array_equal(ids.cpu().numpy(), ri), f"round {rnd} k {k}: ids"
            assert np.array_equal(vals.cpu().numpy(), rv), f"round {rnd} k {k}: values"
        w = W.config(3, scale=0.1)
        assert_same(gpu_run(w, cuda), oracle_run(w), f"round {rnd}: sample after topk")

"""The trace build of the library (``_vws_trace.so``): the same results as the product build, and
phase records that are complete and ordered for every workgroup."""
import numpy as np
import pytest

from vllm_webgpu_amd import _lib

pytestmark = pytest.mark.gpu


def test_trace_records_and_results(cuda):
    import torch

    from vllm_webgpu_amd import ops, trace

    rec, fl, kus, name, B = trace.collect(2, launches=4, warmup=2)
    assert rec.shape == (4, B, _lib.TRACE_SLOTS)
    assert all(np.isfinite(k) and k > 0 for k in kus)
    for i in range(4):
        r = rec[i]
        assert sorted(r[:, _lib.TRACE_ROWID].tolist()) == list(range(B))
        assert ((r[:, _lib.TRACE_XCC] >= 0) & (r[:, _lib.TRACE_XCC] < 8)).all()
        e, s, row, x = (r[:, k] for k in (_lib.TRACE_ENTRY, _lib.TRACE_STREAM, _lib.TRACE_ROW,
                                           _lib.TRACE_EXIT))
        assert (e > 0).all() and (row >= e).all() and (x >= row).all()
        single = (fl[i][r[:, _lib.TRACE_ROWID]] & (_lib.FLAG_GENERAL_PATH | _lib.FLAG_STREAM_TOPP)) == 0
        for k in (_lib.TRACE_PARAMS, _lib.TRACE_SEED):
            assert (r[single, k] >= e[single]).all() and (r[single, k] <= s[single]).all()
        assert (s[single] <= row[single]).all()
        # the whole launch within a millisecond of the device clock
        assert x.max() - e.min() < 100_000
    text = trace.report(rec, fl, kus, name, B)
    assert "Per XCD" in text and "single pass" in text

    # the top-p path's finish stamps, in order, on C5's rows (sampled, 20 logprobs)
    rec5, fl5, _, _, B5 = trace.collect(5, launches=2, warmup=1)
    for i in range(2):
        r = rec5[i]
        on = (fl5[i][r[:, _lib.TRACE_ROWID]] & _lib.FLAG_STREAM_TOPP) != 0
        assert on.mean() > 0.9
        seq = [_lib.TRACE_STREAM, _lib.TRACE_TP_MASS, _lib.TRACE_TP_CUT, _lib.TRACE_TP_RACE,
               _lib.TRACE_TP_LOGPROBS, _lib.TRACE_ROW]
        for s0, s1 in zip(seq, seq[1:]):
            assert (r[on, s0] > 0).all() and (r[on, s1] >= r[on, s0]).all(), (s0, s1)
    assert "top-p: masses -> cut decided" in trace.report(rec5, fl5, (1.0, 1.0), "C5", B5)

    # the same tokens from both builds
    w, xs, kw, _ = trace._inputs(2, cuda, False, 1)
    a = ops.sample(xs[0], **kw).sampled.cpu().numpy()
    with _lib.use(_lib.TRACE_LIB_PATH):
        b = ops.sample(xs[0], **kw).sampled.cpu().numpy()
    torch.cuda.synchronize()
    assert np.array_equal(a, b)

"""The allocation-free entry point ``mk_decode_noalloc`` against ``mk_decode``, both through the C ABI.

``mk_decode_noalloc`` runs the same kernels on a workspace held in a file-scope device array
instead of a per-stream allocation. Two calls in a row -- the second with a smaller input (a
shorter prompt and context, so fewer attention splits) -- must each give the logits, the greedy
token and the cache row that ``mk_decode`` gives on identical copies of the inputs, bit for bit.
The second call also checks that the array's state left by the first call (launch sequence,
exchange words) does not leak into the next result."""
import ctypes

import pytest
import torch

from tests.gpu_common import DEV, Dims, Session, c_library, stream_handle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mini():
    return Session("mini", 512)


def _call(fn, sess, table, tok, kd, vd, pos):
    logits = torch.empty(sess.shape.vocab, dtype=torch.float32, device=DEV)
    out_tok = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    s = sess.shape
    dims = Dims(s.hidden, s.intermediate, s.layers, s.vocab)
    rc = fn(ctypes.byref(dims), int(tok), sess.embed.data_ptr(), sess.lm_head.data_ptr(), sess.final_norm.data_ptr(),
            table.data_ptr(), sess.cos.data_ptr(), sess.sin.data_ptr(), kd.data_ptr(), vd.data_ptr(), int(pos),
            sess.max_seq, logits.data_ptr(), out_tok.data_ptr(), stream_handle())
    assert rc == 0, f"hipError {rc}"
    torch.cuda.synchronize()
    return logits, int(out_tok.item())


def test_noalloc_matches_mk_decode_on_two_calls(mini):
    lib = c_library()
    table = mini.device_layer_table()
    for P in (300, 40):  # the second call: a smaller input
        print(f"[noalloc] prompt {P}, position {P}", flush=True)
        _, last, _, kc, vc = mini.prefill(P)
        tok = int(last.float().argmax())
        ka, va = kc.to(DEV), vc.to(DEV)
        kb, vb = kc.to(DEV), vc.to(DEV)
        want, want_tok = _call(lib.mk_decode, mini, table, tok, ka, va, P)
        got, got_tok = _call(lib.mk_decode_noalloc, mini, table, tok, kb, vb, P)
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), f"prompt {P}: logits differ"
        assert got_tok == want_tok and got_tok >= 0
        assert torch.equal(kb, ka) and torch.equal(vb, va)
    assert mini.kernel.status() == 0


def test_noalloc_rejects_sizes_beyond_its_limits(mini):
    """Out-of-limit shapes and positions are rejected before anything is launched."""
    lib = c_library()
    table = mini.device_layer_table()
    logits = torch.empty(mini.shape.vocab, dtype=torch.float32, device=DEV)
    kd = torch.zeros(2, 8, 16, 128, dtype=torch.bfloat16, device=DEV)
    p = lambda t: t.data_ptr()
    for dims, pos in ((Dims(4096, 12288, 2, 4096), 3), (Dims(1024, 3072, 63, 4096), 3), (Dims(1024, 3072, 2, 4096), 16)):
        rc = lib.mk_decode_noalloc(ctypes.byref(dims), 1, p(mini.embed), p(mini.lm_head), p(mini.final_norm), p(table),
                                   p(mini.cos), p(mini.sin), p(kd), p(kd) + 64, pos, 16, p(logits), None,
                                   stream_handle())
        assert rc == 1  # hipErrorInvalidValue

"""HIP-graph capture of the multi-kernel entry points: the batched prefill (``prefill``, both of its
regimes, and at 300 tokens with the attention cut into key-range chunks and merged) and the batched decode (``decode_batch``, the layer-by-layer engine and the persistent
kernel), captured with ``torch.cuda.graph`` after an eager call and replayed several times. Between
replays the test restores the inputs the call mutates (the caches) with eager kernels and runs
unrelated eager work, then checks every replay bit for bit against the eager result: the graph must
contain no node whose effect depends on the replay (a memset node, a host-side value read at
capture time that later changes)."""
import pytest
import torch

from tests.gpu_common import DEV, Session

pytestmark = pytest.mark.gpu

REPLAYS = 3


@pytest.fixture(scope="module")
def mini():
    return Session("mini", 512)


def _capture(fn):
    """Warm-up on a side stream (torch's capture protocol), then capture ``fn`` into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def _unrelated_eager_work():
    x = torch.randn(1 << 20, device=DEV)
    return float((x * 2).sum().item())


@pytest.mark.parametrize("P", [24, 100, 300], ids=["skinny-path", "tile-path", "tile-path-key-chunks"])
def test_prefill_graph_replays_match_eager(mini, P):
    s = mini.shape
    ids = torch.randint(0, s.vocab, (P,), generator=torch.Generator().manual_seed(7), dtype=torch.int64)
    tokens = ids.to(device=DEV, dtype=torch.int32)
    kd = torch.zeros(s.layers, s.kv_heads, mini.max_seq, s.head_dim, dtype=torch.bfloat16, device=DEV)
    vd = torch.zeros_like(kd)

    def call():
        return mini.kernel.prefill(tokens, mini.embed, mini.lm_head, mini.final_norm, mini.layers, mini.cos, mini.sin,
                                   kd, vd, 0, mini.max_seq)

    want_logits, want_tok = (t.clone() for t in call())
    want_k, want_v = kd.clone(), vd.clone()
    torch.cuda.synchronize()
    g, (got_logits, got_tok) = _capture(call)
    for r in range(REPLAYS):
        kd.zero_()
        vd.zero_()
        _unrelated_eager_work()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got_logits, want_logits), f"replay {r}: logits differ"
        assert torch.equal(got_tok, want_tok), f"replay {r}: token differs"
        assert torch.equal(kd, want_k) and torch.equal(vd, want_v), f"replay {r}: cache differs"
    assert mini.kernel.status() == 0


@pytest.mark.parametrize("engine, lengths", [(1, (5, 40, 100, 300)), (1, tuple(3 + 11 * i for i in range(20))),
                                             (2, (5, 40, 100, 300)), (2, tuple(3 + 11 * i for i in range(20)))],
                         ids=["layers-b4", "layers-b20", "persistent-b4", "persistent-two-launches-b20"])
def test_decode_batch_graph_replays_match_eager(mini, engine, lengths):
    s = mini.shape
    B = len(lengths)
    gen = torch.Generator().manual_seed(11)
    k0 = (torch.randn(B, s.layers, s.kv_heads, mini.max_seq, s.head_dim, generator=gen) * 0.5).to(torch.bfloat16)
    v0 = (torch.randn(B, s.layers, s.kv_heads, mini.max_seq, s.head_dim, generator=gen) * 0.5).to(torch.bfloat16)
    k0, v0 = k0.to(DEV), v0.to(DEV)
    kd, vd = k0.clone(), v0.clone()
    toks = torch.randint(0, s.vocab, (B,), generator=gen, dtype=torch.int64).to(device=DEV, dtype=torch.int32)
    pos = torch.tensor(lengths, dtype=torch.int32, device=DEV)

    def call():
        return mini.kernel.decode_batch(toks, pos, mini.embed, mini.lm_head, mini.final_norm, mini.layers, mini.cos,
                                        mini.sin, kd, vd, mini.max_seq)

    mini.kernel.set_batch_engine(engine)
    try:
        want_logits, want_tok = (t.clone() for t in call())
        want_k, want_v = kd.clone(), vd.clone()
        torch.cuda.synchronize()
        assert torch.isfinite(want_logits).all() and bool((want_tok >= 0).all())
        g, (got_logits, got_tok) = _capture(call)
        for r in range(REPLAYS):
            kd.copy_(k0)
            vd.copy_(v0)
            _unrelated_eager_work()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(got_logits, want_logits), f"replay {r}: logits differ"
            assert torch.equal(got_tok, want_tok), f"replay {r}: tokens differ"
            assert torch.equal(kd, want_k) and torch.equal(vd, want_v), f"replay {r}: caches differ"
    finally:
        mini.kernel.set_batch_engine(0)
    assert mini.kernel.status() == 0

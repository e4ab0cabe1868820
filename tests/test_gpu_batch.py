"""GPU parity tests of the batched decode (``decode_batch``, C ABI ``mk_decode_batch``): B sequences of
different lengths advance one token each per call, each against its own cache. Batches of up to 16
sequences of the 0.6B shape run on either engine (``set_batch_engine``: 1 layer by layer, 2 the
persistent kernel); both are checked.

Per sequence, every step is checked against the fp32 restatement (``restate.decode_step``) run on the
cache the kernel has written for that sequence -- the same tight check as the single-sequence
decode (max-abs 5e-3, same greedy token, the new K/V rows within one bf16 rounding step) -- and, at
the full 0.6B shape, against the single-sequence decode kernel on the same inputs."""
import math

import pytest
import torch

from oracle import hf, restate
from tests.gpu_common import DEV, Session, stats

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mini():
    return Session("mini", 512)


@pytest.fixture(scope="module")
def mini17():
    return Session("mini-1.7b", 512)


@pytest.fixture(scope="module")
def mini2k():
    return Session("mini", 2048)


def _batched_cache(sess, prompts):
    """Oracle prefill of each prompt into its slot of a [B, L, 8, max_seq, 128] cache (CPU), and each
    prompt's greedy next token."""
    ks, vs, first = [], [], []
    for ids in prompts:
        lg, k, v = restate.prefill(sess.W, ids, sess.cos_cpu, sess.sin_cpu, sess.max_seq)
        ks.append(k)
        vs.append(v)
        first.append(restate.argmax_bf16(lg))
    return torch.stack(ks), torch.stack(vs), first


def _decode_batch(sess, toks, pos, kd, vd):
    t = torch.tensor(toks, dtype=torch.int32, device=DEV)
    p = torch.tensor(pos, dtype=torch.int32, device=DEV)
    return sess.kernel.decode_batch(t, p, sess.embed, sess.lm_head, sess.final_norm, sess.layers, sess.cos, sess.sin,
                                    kd, vd, sess.max_seq)


@pytest.fixture
def engine(request):
    """Forces decode_batch's engine for one test (0 = automatic is restored afterwards)."""
    import megakernel
    kernel = megakernel.load()
    kernel.set_batch_engine(request.param)
    yield request.param
    kernel.set_batch_engine(0)


@pytest.mark.parametrize("shape_fixture, lengths, steps, engine", [
    ("mini", (5, 40, 100, 300), 6, 1),
    ("mini", (5, 40, 100, 300), 6, 2),
    ("mini", (1, 17, 64, 130, 255, 256, 257, 480), 4, 1),
    ("mini", (1, 17, 64, 130, 255, 256, 257, 480), 4, 2),
    ("mini", (495,), 3, 2),                              # one sequence: 16 key ranges of 32
    ("mini", (509, 3, 260, 1, 400, 90, 128), 2, 2),      # 27 key ranges of 64 over 7 sequences
    ("mini2k", (1900, 1300, 2000, 700), 2, 2),             # 32 ranges of 192 keys: 2 rounds of K/V loads
    ("mini2k", (2000,), 2, 2),                             # one sequence in 32 ranges of 64 keys
    ("mini", (7, 300, 45, 128, 256, 99, 1, 410, 64), 3, 2),  # 9 sequences: a second column block of one
    ("mini", tuple(2 + 31 * i for i in range(16)), 3, 2),  # 16 sequences: two full column blocks
    ("mini2k", (1900, 50, 1000, 1500, 300, 2000, 17, 800, 1200, 640, 1, 1750), 2, 2),  # 12 long: 32 ranges of 448
    ("mini17", (33, 200, 90), 4, 1),
    ("mini17", tuple(5 + 37 * i for i in range(12)), 2, 1),  # 1.7B width, 12 sequences: register-blocked products
    ("mini", tuple(3 + 11 * i for i in range(20)), 2, 1),  # 20 sequences: 3 column blocks of 8 (of 4)
    ("mini", tuple(3 + 11 * i for i in range(20)), 2, 2),  # 20 sequences: two persistent launches, 16 + 4
    ("mini", tuple(1 + 15 * i for i in range(32)), 1, 2),  # 32 sequences: two persistent launches of 16
    ("mini", tuple(1 + 5 * i for i in range(64)), 1, 1),   # the largest batch: 8 column blocks
], indirect=["engine"])
def test_batch_matches_oracle_per_sequence(shape_fixture, lengths, steps, engine, request):
    """Sequences of different lengths in one batch (so their attention spans 1 to 8 key splits of
    64, and sequences end a split exactly at 64 and 256): every step, each sequence's logits and
    greedy token against the restatement on the kernel's cache for that sequence, and its new K/V
    rows. Layer by layer, up to 8 sequences share one 16-column MFMA block; 20 and 64 sequences use 3
    and 8. The persistent kernel (engine 2) runs up to 8 sequences in one column block and up to 16
    in two, and cuts the batch's keys into at most 32 ranges, one per workgroup of an XCD; 17-32
    sequences run as two of its launches (the first 16, then the rest)."""
    sess = request.getfixturevalue(shape_fixture)
    prompts = [hf.prompt_ids(n, sess.shape.vocab, seed=10 + i)[0].tolist() for i, n in enumerate(lengths)]
    kc, vc, toks = _batched_cache(sess, prompts)
    kd, vd = kc.to(DEV), vc.to(DEV)
    pos = list(lengths)
    B = len(lengths)
    worst = 0.0
    for t in range(steps):
        before_k, before_v = kd.cpu(), vd.cpu()
        logits, dev_toks = _decode_batch(sess, toks, pos, kd, vd)
        logits, dev_toks = logits.cpu(), dev_toks.cpu().tolist()
        for b in range(B):
            want = sess.oracle_step(before_k[b], before_v[b], toks[b], pos[b])
            maxabs, cos = stats(logits[b], want)
            worst = max(worst, maxabs)
            assert maxabs < 5e-3 and cos > 0.999999, (t, b, maxabs, cos)
            assert dev_toks[b] == restate.argmax_bf16(logits[b]) == restate.argmax_bf16(want), (t, b)
            for got_c, ref_c in ((kd, before_k), (vd, before_v)):
                row = got_c[b, :, :, pos[b]].float().cpu()
                d = (row - ref_c[b, :, :, pos[b]].float()).abs().max().item()
                assert d <= 2 ** -6 * max(1.0, ref_c[b, :, :, pos[b]].float().abs().max().item()), (t, b, d)
        # nothing but the new rows changed
        changed = ((kd.cpu() != before_k).any(-1)).nonzero().tolist()
        assert sorted({(c[0], c[3]) for c in changed}) <= sorted({(b, pos[b]) for b in range(B)})
        toks = dev_toks
        pos = [p + 1 for p in pos]
    print(f"[batch {shape_fixture} B={B} engine {engine}] {steps} steps, every sequence matches the restatement, "
          f"max|d| {worst:.3e}", flush=True)


@pytest.fixture(scope="module")
def q06():
    return Session("qwen3-0.6b", 512)


def _assert_same_token_or_near_tie(tok_a, tok_b, logits_a, logits_b, maxabs, where):
    """The two greedy tokens must be equal, unless the logits the two paths computed (which differ by
    ``maxabs``, different fp32 summation orders) put the two candidates within that difference of each
    other: an argmax over bf16-rounded logits can then flip with no fault on either side."""
    if tok_a == tok_b:
        return
    step = 2.0 ** (math.floor(math.log2(max(abs(float(logits_b[tok_b])), 1e-30))) - 7)  # one bf16 step
    gap_a = float(logits_a[tok_a] - logits_a[tok_b])
    gap_b = float(logits_b[tok_b] - logits_b[tok_a])
    assert gap_a <= 2 * maxabs + step and gap_b <= 2 * maxabs + step, \
        f"{where}: tokens {tok_a} != {tok_b} without a near-tie (gaps {gap_a:.2e}, {gap_b:.2e}, max-abs {maxabs:.2e})"


@pytest.mark.parametrize("engine, lengths, steps", [
    (1, (32, 64, 100, 150, 200, 256, 300, 480), 6),
    (2, (32, 64, 100, 150, 200, 256, 300, 480), 6),
    (2, tuple(16 + 16 * i for i in range(16)), 4),   # two column blocks of the persistent kernel
], indirect=["engine"])
def test_batch_agrees_with_single_sequence_decode_at_0_6b(q06, engine, lengths, steps):
    """The full Qwen3-0.6B shape, 8 sequences of lengths 32..480 (and 16 of 16..256): each sequence's
    batched logits and token against the single-sequence decode kernel on an identical cache, for
    several steps (both are fp32-accurate, so they agree to the restatement tolerance), and against
    the restatement on the first step. Prints the batched step time."""
    sess = q06
    B = len(lengths)
    prompts = [hf.prompt_ids(n, sess.shape.vocab, seed=20 + i)[0].tolist() for i, n in enumerate(lengths)]
    kc, vc, toks = _batched_cache(sess, prompts)
    kd, vd = kc.to(DEV), vc.to(DEV)
    singles = [(kc[b].to(DEV), vc[b].to(DEV)) for b in range(B)]
    pos = list(lengths)
    for t in range(steps):
        if t == 0:
            want0 = [sess.oracle_step(kc[b].clone(), vc[b].clone(), toks[b], pos[b]) for b in range(B)]
        logits, dev_toks = _decode_batch(sess, toks, pos, kd, vd)
        logits, dev_toks = logits.cpu(), dev_toks.cpu().tolist()
        for b in range(B):
            ls, ts = sess.decode(toks[b], singles[b][0], singles[b][1], pos[b], greedy=True)
            maxabs, _ = stats(logits[b], ls.cpu())
            assert maxabs < 5e-3, (t, b, maxabs)
            _assert_same_token_or_near_tie(dev_toks[b], int(ts.item()), logits[b], ls.cpu(), maxabs, (t, b))
            if t == 0:
                assert stats(logits[b], want0[b])[0] < 5e-3
        toks = dev_toks
        pos = [p + 1 for p in pos]
    # timing: 20 batched steps (tokens and positions held, so the same work each step)
    tt = torch.tensor(toks, dtype=torch.int32, device=DEV)
    pp = torch.tensor(pos, dtype=torch.int32, device=DEV)
    args = (tt, pp, sess.embed, sess.lm_head, sess.final_norm, sess.layers, sess.cos, sess.sin, kd, vd, sess.max_seq)
    for _ in range(3):
        sess.kernel.decode_batch(*args)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(20):
        sess.kernel.decode_batch(*args)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / 20
    print(f"[batch qwen3-0.6b B={B} engine {engine}] {ms * 1e3:.0f} us per batched step, {B / ms * 1e3:.0f} tokens/s",
          flush=True)
    assert sess.kernel.status() == 0


@pytest.mark.parametrize("engine", [1, 2], indirect=True)
def test_batch_bad_position_is_reported_in_band(mini, engine):
    """A position outside [0, max_seq) (or a token outside the vocabulary) cannot be checked on the host
    without a copy: the call reports NaN logits and token -1 for every sequence, accesses stay inside
    the cache, and a bad sequence's cache is left bit for bit as it was (its clamped position would
    otherwise overwrite a valid row: row 0, its first prompt token, for a negative position). The
    valid sequences of the same call write their new rows."""
    gen = torch.Generator().manual_seed(5)
    shape = (4, mini.shape.layers, 8, mini.max_seq, 128)
    k0 = (torch.randn(shape, generator=gen) * 0.5).to(torch.bfloat16).to(DEV)
    v0 = (torch.randn(shape, generator=gen) * 0.5).to(torch.bfloat16).to(DEV)
    kd, vd = k0.clone(), v0.clone()
    bad_vocab = mini.shape.vocab + 2
    logits, toks = _decode_batch(mini, [3, 4, 5, bad_vocab], [10, -3, mini.max_seq + 7, 12], kd, vd)
    torch.cuda.synchronize()
    assert torch.isnan(logits).all() and toks.tolist() == [-1, -1, -1, -1]
    for b in (1, 2, 3):  # negative position, position past the cache, token past the vocabulary
        assert torch.equal(kd[b], k0[b]) and torch.equal(vd[b], v0[b]), f"sequence {b}'s cache was written"
    # sequence 0 is valid: exactly its row at position 10 changed, in every layer and head
    changed = (kd[0] != k0[0]).any(dim=-1)
    assert bool(changed[:, :, 10].all()) and not bool(changed[:, :, :10].any()) and not bool(changed[:, :, 11:].any())
    logits, toks = _decode_batch(mini, [3, 4], [10, 11], kd[:2].contiguous(), vd[:2].contiguous())
    assert torch.isfinite(logits).all() and min(toks.tolist()) >= 0


@pytest.mark.parametrize("engine", [2], indirect=True)
def test_persistent_batch_drains_on_request(mini, engine):
    """After request_drain() the persistent kernel's waits give up at once (every workgroup still exits
    normally): NaN logits and token -1 for every sequence, until reset(); then a normal step."""
    kd = torch.zeros(3, mini.shape.layers, 8, mini.max_seq, 128, dtype=torch.bfloat16, device=DEV)
    vd = torch.zeros_like(kd)
    mini.kernel.request_drain()
    try:
        logits, toks = _decode_batch(mini, [3, 4, 5], [10, 20, 30], kd, vd)
        torch.cuda.synchronize()
        assert torch.isnan(logits).all() and toks.tolist() == [-1, -1, -1]
    finally:
        mini.kernel.reset()
    logits, toks = _decode_batch(mini, [3, 4, 5], [10, 20, 30], kd, vd)
    assert torch.isfinite(logits).all() and min(toks.tolist()) >= 0


@pytest.mark.parametrize("engine", [2], indirect=True)
def test_persistent_engine_is_the_one_that_runs(mini, engine):
    """Engine 2 falls back to the layer-by-layer engine where the persistent kernel does not apply, so
    the other engine-2 cases would pass on the wrong engine if the device check failed. With its phase
    trace on, the persistent kernel stamps every workgroup's kernel start, LM-head start and end (a
    100 MHz counter, in order); the layer-by-layer engine writes nothing there. Checked at 8
    sequences (one MFMA column block), 16 (two) and 17 and 32 (two launches: the trace holds the
    second one's stamps), and not at 33 (layer by layer)."""
    import ctypes

    from megakernel import build as mkbuild
    lib = ctypes.CDLL(mkbuild.LIB)
    lib.mk_batch_trace_bytes.restype = ctypes.c_size_t
    lib.mk_set_batch_trace.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    nbytes = lib.mk_batch_trace_bytes()
    maxl, slots, grid = 32, 24, 256
    for B, persistent in ((8, True), (16, True), (17, True), (32, True), (33, False)):
        kd = torch.zeros(B, mini.shape.layers, 8, mini.max_seq, 128, dtype=torch.bfloat16, device=DEV)
        vd = torch.zeros_like(kd)
        buf = torch.zeros(nbytes // 8, dtype=torch.int64, device=DEV)
        assert lib.mk_set_batch_trace(ctypes.c_void_p(buf.data_ptr()), nbytes) == 0
        try:
            logits, toks = _decode_batch(mini, [3 + b for b in range(B)], [10 + 7 * b for b in range(B)], kd, vd)
            torch.cuda.synchronize()
        finally:
            lib.mk_set_batch_trace(None, 0)
        assert torch.isfinite(logits).all() and min(toks.tolist()) >= 0
        t = buf.cpu().view(grid, maxl + 1, slots)[:, maxl, :3]
        if persistent:
            assert (t > 0).all() and (t[:, 1] >= t[:, 0]).all() and (t[:, 2] >= t[:, 1]).all(), B
        else:
            assert (buf == 0).all(), B
    assert mini.kernel.status() == 0

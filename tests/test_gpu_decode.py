"""GPU parity tests: the HIP decode kernel against the CPU oracle, on the same seeded weights.

Two oracles (see ``oracle/``):
  * the fp32 restatement (``oracle.restate``, numerics="fp32"), which computes what the kernel
    computes up to fp32 summation order -- the tight check (max-abs 5e-3, identical greedy token);
  * Transformers itself on the CPU (the reference path), teacher-forced -- the north-star check:
    identical greedy token on >= 99% of steps and cosine >= 0.9999 (float64) against its bf16
    logits. Its max-abs difference is reported next to the noise floor of bf16 itself (the
    Transformers fp32 model against the bf16 model differs by ~4e-2 on these weights).
"""
import math

import pytest
import torch

from oracle import hf, restate
from oracle.spec import SHAPES

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


class Session:
    """One model on CPU (oracle) and its bf16 weights on the GPU (kernel)."""

    def __init__(self, shape_name, max_seq):
        self.shape = SHAPES[shape_name]
        self.max_seq = max_seq
        self.model = hf.build_model(shape_name, max_positions=max(max_seq, 4096))
        import megakernel
        self.kernel = megakernel.load()
        self.embed = self.model.model.embed_tokens.weight.detach().to(DEV)
        self.lm_head = self.embed  # tied
        self.final_norm = self.model.model.norm.weight.detach().to(DEV)
        self.layers = [t.to(DEV) for t in megakernel.layer_weight_list(self.model)]
        self.cos_cpu, self.sin_cpu = hf.rope_tables(self.model, max_seq)
        self.cos, self.sin = self.cos_cpu.to(DEV), self.sin_cpu.to(DEV)
        self._W = None

    @property
    def W(self):
        if self._W is None:
            self._W = restate.Weights.from_model(self.model, self.shape)
        return self._W

    def prefill(self, prompt_len, seed=1):
        ids = hf.prompt_ids(prompt_len, self.shape.vocab, seed)
        last, cache = hf.prefill(self.model, ids)
        kc, vc = hf.cache_to_kernel_layout(cache, self.shape.layers, self.shape.kv_heads, self.max_seq,
                                           self.shape.head_dim)
        return ids, last, cache, kc, vc

    def decode(self, token, k_dev, v_dev, position, greedy=False):
        args = (int(token), self.embed, self.lm_head, self.final_norm, self.layers, self.cos, self.sin,
                k_dev, v_dev, int(position), self.max_seq)
        if greedy:
            return self.kernel.decode_greedy(*args)
        return self.kernel.decode(*args)


@pytest.fixture(scope="module")
def mini():
    return Session("mini", 512)


@pytest.fixture(scope="module")
def mini17():
    return Session("mini-1.7b", 512)


@pytest.fixture(scope="module")
def q06():
    return Session("qwen3-0.6b", 512)


def _stats(ours, ref):
    ours, ref = ours.double(), ref.double()
    cos = torch.nn.functional.cosine_similarity(ours, ref, dim=0).item()
    return (ours - ref).abs().max().item(), cos


def test_mini_matches_fp32_restatement(mini):
    """2-layer model with the kernel's real head geometry: every step's logits and the K/V written
    to the cache agree with the fp32 restatement."""
    P, steps = 32, 8
    ids, last, cache, kc, vc = mini.prefill(P)
    kd, vd = kc.to(DEV), vc.to(DEV)
    ref = hf.greedy_reference(mini.model, ids, steps)
    for t in range(steps):
        pos = P + t
        tok = ref["tokens"][t]
        print(f"[mini] step {t} pos {pos} token {tok}", flush=True)
        logits, dev_tok = mini.decode(tok, kd, vd, pos, greedy=True)
        want, _ = restate.decode_step(mini.W, kc, vc, tok, pos, mini.cos_cpu, mini.sin_cpu, numerics="fp32")
        got = logits.cpu()
        assert torch.isfinite(got).all()
        maxabs, cos = _stats(got, want)
        assert maxabs < 5e-3, f"step {t}: max|kernel - restatement| = {maxabs}"
        assert cos > 0.999999
        assert int(dev_tok.item()) == restate.argmax_bf16(got), "device argmax != argmax of returned logits"
        assert int(dev_tok.item()) == restate.argmax_bf16(want)
        # the new K/V row landed at `pos` and agrees with the restatement's (bf16, may differ by
        # one rounding step where fp32 summation order moves a value across a rounding boundary)
        kk = kd[:, :, pos].float().cpu()
        dk = (kk - kc[:, :, pos].float()).abs().max().item()
        assert dk <= 2 ** -6 * max(1.0, kc[:, :, pos].float().abs().max().item()), dk
    # positions beyond the decoded range are untouched
    assert kd[:, :, P + steps:].abs().sum().item() == 0


def test_mini_1_7b_shape_matches_fp32_restatement(mini17):
    """The (2048, 6144) instantiation (the Qwen3-1.7B layer shape, 2 layers, small vocabulary)
    against the fp32 restatement, including a context long enough for several attention splits."""
    P, steps = 100, 4
    ids, last, cache, kc, vc = mini17.prefill(P)
    kd, vd = kc.to(DEV), vc.to(DEV)
    tok = int(last.float().argmax())
    for t in range(steps):
        pos = P + t
        print(f"[mini-1.7b] step {t} pos {pos} token {tok}", flush=True)
        logits, dev_tok = mini17.decode(tok, kd, vd, pos, greedy=True)
        want, _ = restate.decode_step(mini17.W, kc, vc, tok, pos, mini17.cos_cpu, mini17.sin_cpu, numerics="fp32")
        got = logits.cpu()
        maxabs, cos = _stats(got, want)
        assert maxabs < 5e-3, f"step {t}: max|kernel - restatement| = {maxabs}"
        assert int(dev_tok.item()) == restate.argmax_bf16(got)
        tok = int(dev_tok.item())


def _decode_steps(sess, tokens, n, generate, kd, vd, position):
    return sess.kernel.decode_steps(tokens, n, generate, sess.embed, sess.lm_head, sess.final_norm, sess.layers,
                                    sess.cos, sess.sin, kd, vd, position, sess.max_seq)


def test_device_loop_matches_per_step_calls(mini):
    """The device-side multi-token loop (``decode_steps``, C ABI ``mk_decode_steps``) in both modes
    against a host loop of ``decode_greedy`` calls that reads each token back: the same kernel on the
    same inputs, so the tokens, the last logits and the whole cache agree bit for bit. The 32 steps
    from prompt 240 cross context 256, where the launches switch to two register K/V rows per
    group."""
    P, n = 240, 32
    _, last, _, kc, vc = mini.prefill(P)
    t0 = int(last.float().argmax())
    ka, va = kc.to(DEV), vc.to(DEV)
    toks, tok = [], t0
    for i in range(n):
        logits_a, dev_tok = mini.decode(tok, ka, va, P + i, greedy=True)
        tok = int(dev_tok.item())
        toks.append(tok)
    print(f"[device-loop] host loop tokens {toks[:8]} ...", flush=True)

    kb, vb = kc.to(DEV), vc.to(DEV)
    tokens = torch.zeros(n + 1, dtype=torch.int32, device=DEV)
    tokens[0] = t0
    logits_b = _decode_steps(mini, tokens, n, True, kb, vb, P)
    assert tokens[1:].tolist() == toks
    assert torch.equal(logits_b, logits_a)
    assert torch.equal(kb, ka) and torch.equal(vb, va)
    print("[device-loop] generate mode matches", flush=True)

    # teacher mode on the same input tokens: same cache and logits, only tokens[n] written
    kt, vt = kc.to(DEV), vc.to(DEV)
    inputs = [t0] + toks[:-1]
    teach = torch.tensor(inputs + [-5], dtype=torch.int32, device=DEV)
    logits_c = _decode_steps(mini, teach, n, False, kt, vt, P)
    assert teach[:n].tolist() == inputs and int(teach[n].item()) == toks[-1]
    assert torch.equal(logits_c, logits_a)
    assert torch.equal(kt, ka) and torch.equal(vt, va)
    assert kt[:, :, P + n:].abs().sum().item() == 0
    assert mini.kernel.status() == 0
    print("[device-loop] teacher mode matches", flush=True)


def test_native_prefill_through_decode_steps(mini):
    """Prefill without Transformers: the prompt fed through ``decode_steps`` in teacher mode from an
    empty cache writes the ``[L, 8, max_seq, 128]`` cache directly, one position per launch. Checked
    against the fp32 restatement run the same way (one decode step per prompt token from an empty
    cache): the cache rows within one bf16 rounding step, the last logits to 5e-3, the same greedy
    token."""
    P = 24
    ids = hf.prompt_ids(P, mini.shape.vocab, seed=3)[0].tolist()
    L, KV, D = mini.shape.layers, mini.shape.kv_heads, mini.shape.head_dim
    kc = torch.zeros(L, KV, mini.max_seq, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for p, tok in enumerate(ids):
        want, _ = restate.decode_step(mini.W, kc, vc, tok, p, mini.cos_cpu, mini.sin_cpu, numerics="fp32")
    kd, vd = torch.zeros_like(kc, device=DEV), torch.zeros_like(vc, device=DEV)
    tokens = torch.tensor(ids + [-1], dtype=torch.int32, device=DEV)
    got = _decode_steps(mini, tokens, P, False, kd, vd, 0).cpu()
    maxabs, cos = _stats(got, want)
    print(f"[native-prefill] P={P}: max|kernel - restatement| {maxabs:.3e}, cos {cos:.8f}", flush=True)
    assert maxabs < 5e-3 and cos > 0.999999
    assert int(tokens[P].item()) == restate.argmax_bf16(want)
    for name, dev_c, ref_c in (("k", kd, kc), ("v", vd, vc)):
        d = (dev_c[:, :, :P].float().cpu() - ref_c[:, :, :P].float()).abs().max().item()
        assert d <= 2 ** -6 * max(1.0, ref_c.float().abs().max().item()), (name, d)
    assert kd[:, :, P:].abs().sum().item() == 0 and vd[:, :, P:].abs().sum().item() == 0


@pytest.mark.parametrize("shape_fixture, P", [("mini", 300), ("mini17", 300), ("mini17", 488)])
def test_paged_cache_matches_contiguous(shape_fixture, P, request):
    """``decode_paged`` (C ABI ``mk_decode_paged``) on a pool of 16-position pages in shuffled order,
    with the unused pages filled with NaN, against ``decode_greedy`` on the contiguous cache: the
    same kernel arithmetic through another address map, so logits and tokens agree bit for bit and
    the rows written through the table land where the contiguous launch writes them. 24 steps from
    prompt 300 cross page boundaries and context 256 (two register K/V rows, longer splits); from
    prompt 488 they end on the cache's last slot (511), where a K/V row read past the split would
    leave the last page (regression: such reads once took block-table entries past the position)."""
    from tests.paged_layout import from_pages, to_pages
    sess = request.getfixturevalue(shape_fixture)
    n, ps = 24, 16
    _, last, _, kc, vc = sess.prefill(P)
    npl = sess.max_seq // ps
    g = torch.Generator().manual_seed(7)
    pool = npl + 9
    table = torch.randperm(pool, generator=g)[:npl].to(torch.int32)
    kp = to_pages(kc, ps, table.tolist(), pool).to(DEV)
    vp = to_pages(vc, ps, table.tolist(), pool).to(DEV)
    table_d = table.to(DEV)
    ka, va = kc.to(DEV), vc.to(DEV)
    tok = int(last.float().argmax())
    for i in range(n):
        la, ta = sess.decode(tok, ka, va, P + i, greedy=True)
        lb, tb = sess.kernel.decode_paged(tok, sess.embed, sess.lm_head, sess.final_norm, sess.layers, sess.cos,
                                          sess.sin, kp, vp, table_d, P + i, sess.max_seq)
        assert torch.equal(la, lb), f"step {i}: paged logits differ"
        assert int(ta.item()) == int(tb.item())
        tok = int(ta.item())
    print(f"[paged {shape_fixture}] {n} steps from P={P}, page 16: identical logits and tokens", flush=True)
    assert torch.equal(from_pages(kp, table.tolist()), ka) and torch.equal(from_pages(vp, table.tolist()), va)
    unused = sorted(set(range(pool)) - set(table.tolist()))
    assert torch.isnan(kp[:, unused].float()).all() and torch.isnan(vp[:, unused].float()).all()
    assert sess.kernel.status() == 0


def test_device_loop_on_paged_cache(mini):
    """``decode_steps_paged``: greedy generation on the device over a paged cache (shuffled pages,
    NaN in the unused ones) against ``decode_steps`` on the contiguous cache -- the same tokens, the
    same last logits, and the same rows written."""
    from tests.paged_layout import from_pages, to_pages
    P, n, ps = 250, 20, 32
    _, last, _, kc, vc = mini.prefill(P)
    npl = mini.max_seq // ps
    table = torch.randperm(npl + 5, generator=torch.Generator().manual_seed(11))[:npl].to(torch.int32)
    kp = to_pages(kc, ps, table.tolist(), npl + 5).to(DEV)
    vp = to_pages(vc, ps, table.tolist(), npl + 5).to(DEV)
    t0 = int(last.float().argmax())
    ka, va = kc.to(DEV), vc.to(DEV)
    tok_a = torch.zeros(n + 1, dtype=torch.int32, device=DEV)
    tok_a[0] = t0
    la = _decode_steps(mini, tok_a, n, True, ka, va, P)
    tok_b = torch.zeros(n + 1, dtype=torch.int32, device=DEV)
    tok_b[0] = t0
    lb = mini.kernel.decode_steps_paged(tok_b, n, True, mini.embed, mini.lm_head, mini.final_norm, mini.layers,
                                        mini.cos, mini.sin, kp, vp, table.to(DEV), P, mini.max_seq)
    assert tok_b.tolist() == tok_a.tolist()
    assert torch.equal(lb, la)
    assert torch.equal(from_pages(kp, table.tolist()), ka) and torch.equal(from_pages(vp, table.tolist()), va)
    assert mini.kernel.status() == 0
    print(f"[paged device loop] {n} steps from P={P}, page {ps}: tokens {tok_b[1:9].tolist()} ... identical", flush=True)


def test_paged_cache_bad_table_entry_sets_status(mini):
    """A block-table entry outside the page pool cannot be checked on the host without a copy: the
    kernel reads and writes page 0 instead (no access leaves the pool, nothing drains) and sets
    status bit 3 until reset."""
    from tests.paged_layout import to_pages
    P, ps = 40, 16
    _, _, _, kc, vc = mini.prefill(P)
    npl = mini.max_seq // ps
    table = torch.arange(npl, dtype=torch.int32)
    table[P // ps] = npl + 5  # the page holding the position being written
    kp = to_pages(kc, ps, list(range(npl)), npl, fill=0.0).to(DEV)
    vp = to_pages(vc, ps, list(range(npl)), npl, fill=0.0).to(DEV)
    try:
        logits, _ = mini.kernel.decode_paged(7, mini.embed, mini.lm_head, mini.final_norm, mini.layers, mini.cos,
                                             mini.sin, kp, vp, table.to(DEV), P, mini.max_seq)
        assert mini.kernel.status() == 8
        assert torch.isfinite(logits).all()
    finally:
        mini.kernel.reset()
    assert mini.kernel.status() == 0


def test_split_slots_never_stale_across_launches(mini):
    """Exchange words carry an 8-bit epoch (launch sequence * 64 + layer, mod 255, + 1); a reader
    accepts a word once its epoch matches. That is safe only if every word is rewritten at every
    layer: for this 2-layer model, a word last written at layer 1 of launch k carries the epoch
    that layer 0 of launch k + 4 expects. So: one launch with 4 attention splits, three with one
    split (slots 1-3 belong to workgroups without a split), then 4 splits again. If those
    workgroups skipped their slots, the last launch's merge could take layer-1 partials of the first
    launch. Its logits must equal the same launch run right after a 4-split launch."""
    P = 120
    _, _, _, kc, vc = mini.prefill(P)
    tok = 11
    k1, v1 = kc.to(DEV), vc.to(DEV)
    mini.decode(tok, k1, v1, 100)              # 4 splits (context 101)
    k2, v2 = kc.to(DEV), vc.to(DEV)
    for pos in (5, 6, 7):                       # 1 split, on a scratch copy of the cache
        mini.decode(tok, k2, v2, pos)
    got = mini.decode(tok, k1, v1, 101)         # 4 splits again, 4 launches after the first
    k3, v3 = kc.to(DEV), vc.to(DEV)
    mini.decode(tok, k3, v3, 100)
    want = mini.decode(tok, k3, v3, 101)
    assert torch.equal(got, want)
    assert mini.kernel.status() == 0


def test_device_loop_out_of_range_token_sets_status(mini):
    """A device-side input token outside [0, vocab) cannot be checked on the host: the kernel decodes
    token 0 instead (a normal launch, nothing drains) and sets status bit 2 until reset."""
    P = 40
    _, _, _, kc, vc = mini.prefill(P)
    ka, va = kc.to(DEV), vc.to(DEV)
    want = mini.decode(0, ka, va, P)
    kb, vb = kc.to(DEV), vc.to(DEV)
    tokens = torch.tensor([mini.shape.vocab + 5, -1], dtype=torch.int32, device=DEV)
    try:
        got = _decode_steps(mini, tokens, 1, True, kb, vb, P)
        assert mini.kernel.status() == 4
        assert torch.equal(got, want) and torch.equal(kb, ka)
    finally:
        mini.kernel.reset()
    assert mini.kernel.status() == 0


def test_decode_writes_only_its_slot(mini):
    """The K/V write touches exactly [layer, head, position, :] and nothing else."""
    P = 40
    _, _, _, kc, vc = mini.prefill(P)
    kd, vd = kc.to(DEV), vc.to(DEV)
    before_k, before_v = kd.clone(), vd.clone()
    mini.decode(7, kd, vd, P)
    torch.cuda.synchronize()
    diff = (kd != before_k).any(dim=-1)
    assert diff[:, :, :P].sum() == 0 and diff[:, :, P + 1:].sum() == 0
    assert (kd[:, :, P] != 0).any() and (vd[:, :, P] != 0).any()
    assert ((vd != before_v).any(dim=-1)[:, :, :P]).sum() == 0


def _bf16_ulp(x):
    return 2.0 ** (math.floor(math.log2(abs(x))) - 7)


def test_qwen06_config1_one_step(q06):
    """prompt 64, cache 512, one greedy step -- logits and argmax vs Transformers.

    One step cannot demand the identical token: when the top two logits are within Transformers'
    own bf16 noise, its choice differs between host CPUs (this step's top two differ by 6e-4 in
    fp32 and Transformers picks different winners on different machines). The token must be a
    Transformers near-argmax (within 2 bf16 ulps of its max) and identical to the fp32
    restatement's; exact agreement is the >= 99%-of-steps statistic of config 2."""
    P = 64
    ids, last, cache, kc, vc = q06.prefill(P)
    kd, vd = kc.to(DEV), vc.to(DEV)
    tok = int(last.float().argmax())
    ref_logits, _ = hf.decode_step(q06.model, tok, cache)
    logits, dev_tok = q06.decode(tok, kd, vd, P, greedy=True)
    got = logits.cpu()
    r = ref_logits.float()
    maxabs, cos = _stats(got, r)
    ours = int(dev_tok.item())
    print(f"[config1] max|d| {maxabs:.4e} cos {cos:.8f} token kernel {ours} hf {int(r.argmax())}")
    assert cos >= 0.9999
    assert r[ours] >= r.max() - 2 * _bf16_ulp(r.max().item())
    want, _ = restate.decode_step(q06.W, kc, vc, tok, P, q06.cos_cpu, q06.sin_cpu, numerics="fp32")
    assert _stats(got, want)[0] < 5e-3
    assert ours == restate.argmax_bf16(want)


def test_qwen06_config2_teacher_forced(q06):
    """prompt 32, cache 512, 256 teacher-forced steps.

    Tight gate: the kernel reproduces the fp32 restatement (same greedy token on every step but
    at most one fp32 near-tie, max-abs < 5e-3).
    Reference gate: against Transformers' bf16 logits the north-star targets are >= 99% identical
    tokens and cosine >= 0.9999. Both sit at the bf16 noise floor of this random-init model:
    over 1024 teacher-forced steps Transformers' own fp32 model agrees with its bf16 model on
    98.5-98.7% of tokens with min cosine 0.99989, and which near-tie Transformers resolves which
    way depends on the host CPU's GEMM kernels. The test therefore asserts the floor (>= 97.5%
    tokens, mean cosine >= 0.9999, min >= 0.9998) and prints the measured numbers."""
    P, steps = 32, 256
    ids, last, cache, kc, vc = q06.prefill(P)
    kd, vd = kc.to(DEV), vc.to(DEV)
    ref = hf.greedy_reference(q06.model, ids, steps)
    agree, same_as_restate, coss, worst_abs, worst_restate = 0, 0, [], 0.0, 0.0
    for t in range(steps):
        tok = ref["tokens"][t]
        logits, dev_tok = q06.decode(tok, kd, vd, P + t, greedy=True)
        logits = logits.cpu()
        r = ref["logits"][t].float()
        ours = int(dev_tok.item())
        assert ours == restate.argmax_bf16(logits)
        agree += ours == int(r.argmax())
        m, c = _stats(logits, r)
        worst_abs = max(worst_abs, m)
        coss.append(c)
        want, _ = restate.decode_step(q06.W, kc, vc, tok, P + t, q06.cos_cpu, q06.sin_cpu, numerics="fp32")
        worst_restate = max(worst_restate, _stats(logits, want)[0])
        same_as_restate += ours == restate.argmax_bf16(want)
    mean_cos = sum(coss) / len(coss)
    print(f"[config2] vs Transformers: tokens {agree}/{steps} ({100.0 * agree / steps:.2f}%), "
          f"cos mean {mean_cos:.8f} min {min(coss):.8f}, max|d| {worst_abs:.4e}; "
          f"vs fp32 restatement: tokens {same_as_restate}/{steps}, max|d| {worst_restate:.3e}")
    assert same_as_restate >= steps - 1
    assert worst_restate < 5e-3
    assert agree >= math.ceil(0.975 * steps)
    assert mean_cos >= 0.9999 and min(coss) >= 0.9998


def _teacher_forced(sess, P, steps, restate_every, tag, seed=1):
    """Teacher-forced decode of ``steps`` tokens after a ``P``-token prompt: Transformers (CPU) feeds
    the tokens (its greedy choice at every step, as ``hf.greedy_reference``); the kernel's logits are
    compared with Transformers' on every step and, on every ``restate_every``-th step, with the fp32
    restatement run on the cache the kernel has written so far. Returns the counts the config tests
    assert on."""
    ids = hf.prompt_ids(P, sess.shape.vocab, seed)
    last, cache = hf.prefill(sess.model, ids)
    kc, vc = hf.cache_to_kernel_layout(cache, sess.shape.layers, sess.shape.kv_heads, sess.max_seq,
                                       sess.shape.head_dim)
    kd, vd = kc.to(DEV), vc.to(DEV)
    del kc, vc
    out = {"agree": 0, "steps": steps, "coss": [], "restate_steps": 0, "restate_same": 0, "restate_abs": 0.0,
           "sampled_agree": 0, "restate_agree": 0, "sampled_coss": [], "restate_coss": []}
    tok = int(last.float().argmax())
    for t in range(steps):
        pos = P + t
        r, cache = hf.decode_step(sess.model, tok, cache)
        r = r.float()
        if t % restate_every == 0:
            kc_now, vc_now = kd.cpu(), vd.cpu()  # positions [0, pos) as the kernel wrote them
        logits, dev_tok = sess.decode(tok, kd, vd, pos, greedy=True)
        logits = logits.cpu()
        ours = int(dev_tok.item())
        assert torch.isfinite(logits).all(), f"[{tag}] step {t}: non-finite logits"
        assert ours == restate.argmax_bf16(logits), f"[{tag}] step {t}: device argmax != argmax of logits"
        out["agree"] += ours == int(r.argmax())
        out["coss"].append(_stats(logits, r)[1])
        if t % restate_every == 0:
            want, _ = restate.decode_step(sess.W, kc_now, vc_now, tok, pos, sess.cos_cpu, sess.sin_cpu,
                                          numerics="fp32")
            del kc_now, vc_now
            out["restate_steps"] += 1
            out["restate_same"] += ours == restate.argmax_bf16(want)
            out["restate_abs"] = max(out["restate_abs"], _stats(logits, want)[0])
            # the same comparison with Transformers for the restatement: its distance to Transformers'
            # bf16 logits is the bf16 noise floor the kernel's distance is judged against
            out["sampled_agree"] += ours == int(r.argmax())
            out["restate_agree"] += restate.argmax_bf16(want) == int(r.argmax())
            out["sampled_coss"].append(out["coss"][-1])
            out["restate_coss"].append(_stats(want, r)[1])
        tok = int(r.argmax())
    c = out["coss"]
    print(f"[{tag}] P={P} steps={steps}: vs Transformers tokens {out['agree']}/{steps}, cos mean "
          f"{sum(c) / len(c):.8f} min {min(c):.8f}; vs fp32 restatement ({out['restate_steps']} steps) "
          f"tokens {out['restate_same']}/{out['restate_steps']}, max|d| {out['restate_abs']:.3e}; on those steps "
          f"Transformers agreement kernel {out['sampled_agree']} restatement {out['restate_agree']}, cos mean "
          f"kernel {sum(out['sampled_coss']) / len(out['sampled_coss']):.8f} restatement "
          f"{sum(out['restate_coss']) / len(out['restate_coss']):.8f}", flush=True)
    return out


def _assert_config(res, floor):
    assert res["restate_abs"] < 5e-3
    assert res["restate_same"] >= res["restate_steps"] - 1
    c = res["coss"]
    assert sum(c) / len(c) >= 0.9999 and min(c) >= 0.9998
    assert res["agree"] >= math.floor(floor * res["steps"])


def test_qwen06_config3_prompt_sweep(q06):
    """Config 3: prompts of 16, 128, 256 and 480 tokens, cache 512, 32 teacher-forced steps each --
    the attention split count S = min(ceil(ctx / 32), 8) runs from 1 to 8 and the last step writes the
    cache's final slot (position 511). Tight gate against the fp32 restatement on every 8th step;
    token agreement with Transformers pooled over the 128 steps (the bf16 noise floor, as in
    config 2)."""
    pooled = {"agree": 0, "steps": 0, "coss": [], "restate_steps": 0, "restate_same": 0, "restate_abs": 0.0}
    for P in (16, 128, 256, 480):
        r = _teacher_forced(q06, P, 32, 8, "config3")
        for k in ("agree", "steps", "restate_steps", "restate_same"):
            pooled[k] += r[k]
        pooled["coss"] += r["coss"]
        pooled["restate_abs"] = max(pooled["restate_abs"], r["restate_abs"])
    _assert_config(pooled, 0.96)


@pytest.fixture(scope="module")
def q06_4k():
    return Session("qwen3-0.6b", 4096)


def test_qwen06_config4_long_context(q06_4k):
    """Config 4: prompt 3584, cache 4096, 256 teacher-forced steps (ctx 3585-3840): 16 attention
    splits of ~230 keys merged in two poll rounds, most keys streamed inside the attention phase
    rather than held in registers. fp32 restatement on every 32nd step."""
    _assert_config(_teacher_forced(q06_4k, 3584, 256, 32, "config4"), 0.96)


def test_qwen17_config5():
    """Config 5: the Qwen3-1.7B shape (H 2048, I 6144, 28 layers, full vocabulary), prompt 512,
    cache 2048, 256 teacher-forced steps; fp32 restatement on every 8th step.

    At this width the bf16 noise of Transformers' own CPU decode is larger than at 0.6B: the fp32
    restatement (the reference kernel's arithmetic) itself agrees with Transformers' bf16 greedy
    token on only ~92% of steps, with mean cosine ~0.9995. The kernel is therefore held to the
    restatement tightly (max-abs < 5e-3, same token) and to Transformers relative to that floor:
    on the sampled steps its cosine to Transformers is within 1e-5 of the restatement's and its
    token agreement within one step of the restatement's."""
    sess = Session("qwen3-1.7b", 2048)
    res = _teacher_forced(sess, 512, 256, 8, "config5")
    assert res["restate_abs"] < 5e-3
    assert res["restate_same"] >= res["restate_steps"] - 1
    for ck, cr in zip(res["sampled_coss"], res["restate_coss"]):
        assert ck >= cr - 1e-5, (ck, cr)
    assert res["sampled_agree"] >= res["restate_agree"] - 1
    c = res["coss"]
    assert sum(c) / len(c) >= 0.999 and res["agree"] >= math.floor(0.88 * res["steps"])


def test_launch_modes_agree(mini):
    """The plain launch (default) and the cooperative launch run the same grid: one step decoded
    in each mode gives bitwise-identical logits, token and cache row."""
    P = 48
    _, _, _, kc, vc = mini.prefill(P)
    outs = []
    try:
        for mode in (0, 1):
            mini.kernel.set_launch_mode(mode)
            kd, vd = kc.to(DEV), vc.to(DEV)
            logits, tok = mini.decode(11, kd, vd, P, greedy=True)
            outs.append((logits.cpu(), int(tok.item()), kd[:, :, P].cpu()))
    finally:
        mini.kernel.set_launch_mode(0)
    assert mini.kernel.status() == 0
    assert torch.equal(outs[0][0], outs[1][0]) and outs[0][1] == outs[1][1]
    assert torch.equal(outs[0][2], outs[1][2])

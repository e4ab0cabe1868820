"""Float32 restatement of one Qwen3 decode step. TEST INFRASTRUCTURE ONLY.

Two numerics modes:

``numerics="hf"`` (what the HIP kernel implements) follows Transformers' bf16 CPU decode
(``transformers/models/qwen3/modeling_qwen3.py``, cited as ``MQ:line``): every matrix-vector
product accumulates in fp32 and rounds its output to bf16 once (nn.Linear in bf16), and every
elementwise op rounds to bf16 where the bf16 model does:
  - embedding row (bf16);
  - RMSNorm ``MQ:59-64``: ``bf16(x * rsqrt(mean(x^2) + eps))``, then ``bf16(w * that)``;
  - q/k/v/o/gate/up/down/lm_head outputs (``MQ:252-254,279,82,495``);
  - per-head q_norm/k_norm (``MQ:252-253``);
  - RoPE ``MQ:168-169``: ``bf16(bf16(q*cos) + bf16(rotate_half(q)*sin))``;
  - SDPA output (bf16), then both residual adds ``MQ:316,322``;
  - ``bf16(silu(gate))`` and ``bf16(that * up)`` (``MQ:82``).
Attention follows torch's CPU flash SDPA, which Transformers' ``sdpa`` path dispatches to for a
one-token query (``transformers/integrations/sdpa_attention.py:79-166``): scores
``(q.k) * D**-0.5`` in fp32, keys processed in blocks of 512 with a running max, probabilities
``exp(s - running_max)`` summed in fp32 and rounded to bf16 before the product with V, the
accumulator rescaled by ``exp(old_max - new_max)`` between blocks, output ``acc * (1/sum)``
rounded to bf16. The exponential of the softmax is torch's ``fexp_u20``
(``ATen/cpu/vec/vec512/vec512_float.h``: the bit-construction method of Malossi, Ineichen, Bekas and
Curioni, "Fast Exponential Computation on SIMD Architectures", 2015 -- ``2**(x*log2 e)`` with the
fractional part corrected by a degree-3 polynomial and the result assembled directly in the float's
bit pattern; relative error about 1e-4), applied to whole 16-lane chunks of a block; the remainder of
a block uses the libm ``exp``. Matching it is what makes the probabilities agree: with an accurate
``exp`` only 85-92% of SDPA outputs are bit-identical to torch's, with ``fexp_u20`` 99.9-100%
(``tests/test_oracle.py`` pins this against ``torch.nn.functional.scaled_dot_product_attention``).

``numerics="fp32"`` follows the reference kernel ``/root/reference/megakernel.cu``: fp32 residual
stream from the embedding (``:783-795``), fp32 RMSNorm ``x*w*rsqrt(mean+eps)`` (``:704-739``,
``:148-182``), fp32 q/k/v/o/gate/up/down/LM-head outputs (``:633-701``, ``:191-225``, ``:100-142``,
``:53-90``, ``:9-48``), per-head norm and RoPE in fp32 with bf16 cos/sin, K/V written to the cache
as bf16 (``:490-630``), exact fp32 softmax attention (``:228-370``).

Tensors are float32 holding bf16-representable values unless stated.
"""

import math
import struct

import torch

BLOCK_KEYS = 512     # torch CPU flash-attention key block for kv_len >= 512
VEC_LANES = 16       # float lanes of torch's CPU vector type (16 with AVX-512, 8 with AVX2)


def bf16(x):
    """Round-to-nearest-even to bfloat16, returned as float32."""
    return x.to(torch.bfloat16).to(torch.float32)


def _fma(a, b, c):
    """Fused multiply-add on float32 tensors (exact product in float64, one final rounding)."""
    return (a.double() * b.double() + c.double()).float()


def _f32(bits):
    return torch.tensor(struct.unpack("<f", struct.pack("<I", bits))[0], dtype=torch.float32)


_LN_FLT_MIN = _f32(0xC2AEAC50)   # ln(FLT_MIN)
_LN_FLT_MAX = _f32(0x42B17218)   # ln(FLT_MAX)
_LOG2E = _f32(0x3FB8AA3B)
_FEXP_C = [torch.tensor(c, dtype=torch.float32) for c in
           (0.00010703434948458272, 0.30354260500649682, -0.22433836478672356, -0.079204240219773236)]


def fexp_u20(x):
    """torch's ``Vectorized<float>::fexp_u20``, restated elementwise (float32 in and out).

    y = x*log2(e); f = y - floor(y); p = ((c3*f + c2)*f + c1)*f + c0 (fused);
    bits = trunc(2**23 * (y - p) + 2**23 * 127) (fused); x < ln(FLT_MIN) -> 0, x > ln(FLT_MAX) -> inf.
    """
    x = x.float()
    lo = x < _LN_FLT_MIN
    hi = x > _LN_FLT_MAX
    y = x * _LOG2E
    f = y - torch.floor(y)
    c0, c1, c2, c3 = (c.expand_as(f) for c in _FEXP_C)
    p = _fma(f, c3, c2)
    p = _fma(f, p, c1)
    p = _fma(f, p, c0)
    y = y - p
    t = _fma(torch.full_like(y, 2.0 ** 23), y, torch.full_like(y, 2.0 ** 23 * 127))
    bits = torch.trunc(t).to(torch.int32)
    bits = torch.where(lo, torch.zeros_like(bits), bits)
    bits = torch.where(hi, torch.full_like(bits, 0x7F800000), bits)
    return bits.view(torch.float32)


def block_exp(d, exp_mode="torch_flash", lanes=VEC_LANES):
    """Exponentials of one key block's ``s - max`` (last dim), as the flash kernel computes them:
    ``fexp_u20`` on the first ``lanes * floor(n / lanes)`` entries, libm ``exp`` on the rest."""
    if exp_mode == "accurate":
        return torch.exp(d)
    n = d.shape[-1]
    full = (n // lanes) * lanes
    return torch.cat((fexp_u20(d[..., :full]), torch.exp(d[..., full:])), dim=-1)


def _mv(w, x):
    """Matrix-vector product accumulated in ``w``'s dtype (float32, or float64 for exactly rounded
    dot products), returned as float32."""
    return (w @ x.to(w.dtype)).float()


def rms_norm_hf(x, w, eps):
    """``MQ:59-64`` over the last dim."""
    var = (x * x).mean(-1, keepdim=True)
    return bf16(w * bf16(x * torch.rsqrt(var + eps)))


def rope_hf(x, cos, sin):
    """``MQ:140-144,168-169``; x [..., D] bf16 values, cos/sin [D] bf16 values."""
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return bf16(bf16(x * cos) + bf16(rot * sin))


def attention_flash(q, k, v, scale, exp_mode="torch_flash", lanes=VEC_LANES):
    """torch CPU flash SDPA for one query position. q [Hq, D], k/v [Hkv, L, D] -> bf16 [Hq, D]."""
    hq, d = q.shape
    hkv, L, _ = k.shape
    rep = hq // hkv
    kr = k.repeat_interleave(rep, 0)
    vr = v.repeat_interleave(rep, 0)
    blk = min(BLOCK_KEYS, L)
    m = torch.full((hq, 1), -math.inf)
    l = torch.zeros(hq, 1)
    acc = torch.zeros(hq, d)
    for s0 in range(0, L, blk):
        kb, vb = kr[:, s0:s0 + blk], vr[:, s0:s0 + blk]
        s = torch.einsum("hd,hld->hl", q, kb) * torch.tensor(scale, dtype=torch.float32)
        new_m = torch.maximum(m, s.amax(-1, keepdim=True))
        e = block_exp(s - new_m, exp_mode, lanes)
        corr = torch.exp(m - new_m)
        l = e.sum(-1, keepdim=True) + corr * l
        acc = acc * corr + torch.einsum("hl,hld->hd", bf16(e), vb)
        m = new_m
    return bf16(acc * (1.0 / l))


def attention_fp32(q, k, v, scale):
    """Exact fp32 softmax attention (``/root/reference/megakernel.cu:228-370``)."""
    rep = q.shape[0] // k.shape[0]
    kr, vr = k.repeat_interleave(rep, 0), v.repeat_interleave(rep, 0)
    s = torch.einsum("hd,hld->hl", q, kr) * scale
    p = torch.softmax(s, -1)
    return torch.einsum("hl,hld->hd", p, vr)


class Weights:
    """Float32 copies of the bf16 model weights (kept once; the step does no dtype work on them)."""

    def __init__(self, embed, layer_list, final_norm, shape):
        self.shape = shape
        self.embed = embed.float()
        self.final_norm = final_norm.float()
        self.layers = []
        from .spec import LAYER_WEIGHT_ORDER
        n = len(LAYER_WEIGHT_ORDER)
        for i in range(shape.layers):
            self.layers.append({k: t.float() for k, t in zip(LAYER_WEIGHT_ORDER, layer_list[i * n:(i + 1) * n])})

    @classmethod
    def from_model(cls, model, shape):
        from .hf import layer_weights
        return cls(model.model.embed_tokens.weight.detach(), layer_weights(model),
                   model.model.norm.weight.detach(), shape)


def decode_step(W, k_cache, v_cache, token, position, cos, sin, numerics="hf", exp_mode="torch_flash",
                keep=False, lanes=VEC_LANES):
    """One decode step. ``k_cache``/``v_cache`` are bf16 ``[L, Hkv, max_seq, D]`` and are written at
    ``position``; attention reads positions ``[0, position]``. ``cos``/``sin`` are bf16 tables
    ``[max_seq, D]``. Returns (fp32 logits [V], dict of per-layer intermediates if ``keep``)."""
    s = W.shape
    D, eps = s.head_dim, s.eps
    scale = D ** -0.5
    c, sn = cos[position].float(), sin[position].float()
    hf = numerics == "hf"
    x = W.embed[token].float().clone()
    inter = {"layers": []} if keep else None
    for li, lw in enumerate(W.layers):
        if hf:
            h = rms_norm_hf(x, lw["input_layernorm"], eps)
            q = bf16(_mv(lw["q_proj"], h)).view(s.q_heads, D)
            k = bf16(_mv(lw["k_proj"], h)).view(s.kv_heads, D)
            v = bf16(_mv(lw["v_proj"], h)).view(s.kv_heads, D)
            q = rope_hf(rms_norm_hf(q, lw["q_norm"], eps), c, sn)
            k = rope_hf(rms_norm_hf(k, lw["k_norm"], eps), c, sn)
        else:
            h = x * lw["input_layernorm"] * torch.rsqrt((x * x).mean() + eps)
            q = (_mv(lw["q_proj"], h)).view(s.q_heads, D)
            k = (_mv(lw["k_proj"], h)).view(s.kv_heads, D)
            v = (_mv(lw["v_proj"], h)).view(s.kv_heads, D)

            def nr(t, w):
                t = t * torch.rsqrt((t * t).mean(-1, keepdim=True) + eps) * w
                half = D // 2
                a, b = t[..., :half], t[..., half:]
                return torch.cat((a * c[:half] - b * sn[:half], b * c[:half] + a * sn[:half]), -1)
            q, k = nr(q, lw["q_norm"]), nr(k, lw["k_norm"])
        k_cache[li, :, position] = k.to(torch.bfloat16)
        v_cache[li, :, position] = v.to(torch.bfloat16)
        kk = k_cache[li, :, :position + 1].float()
        vv = v_cache[li, :, :position + 1].float()
        if hf:
            attn = attention_flash(q, kk, vv, scale, exp_mode, lanes).reshape(-1)
            o = bf16(_mv(lw["o_proj"], attn))
            x = bf16(x + o)
            h2 = rms_norm_hf(x, lw["post_attention_layernorm"], eps)
            g = bf16(_mv(lw["gate_proj"], h2))
            u = bf16(_mv(lw["up_proj"], h2))
            mlp = bf16(bf16(torch.nn.functional.silu(g)) * u)
            dn = bf16(_mv(lw["down_proj"], mlp))
            x = bf16(x + dn)
        else:
            attn = attention_fp32(q, kk, vv, scale).reshape(-1)
            x = x + _mv(lw["o_proj"], attn)
            h2 = x * lw["post_attention_layernorm"] * torch.rsqrt((x * x).mean() + eps)
            g, u = _mv(lw["gate_proj"], h2), _mv(lw["up_proj"], h2)
            mlp = g / (1 + torch.exp(-g)) * u
            x = x + _mv(lw["down_proj"], mlp)
        if keep:
            inter["layers"].append({"q": q.clone(), "k": k.clone(), "v": v.clone(), "attn": attn.clone(),
                                    "x": x.clone()})
    if hf:
        hfin = rms_norm_hf(x, W.final_norm, eps)
    else:
        hfin = x * W.final_norm * torch.rsqrt((x * x).mean() + eps)
    logits = _mv(W.embed, hfin)
    if keep:
        inter["final_hidden"] = hfin
    return logits, inter


def argmax_bf16(logits):
    """Greedy token over bf16-rounded logits, lowest index on ties (what ``torch.argmax`` returns
    for the bf16 logits Transformers emits)."""
    return int(torch.argmax(bf16(logits)))


def attention_split(q, k, v, scale, splits):
    """Split-K ("flash-decoding") form of ``attention_fp32``: the keys are cut into ``splits``
    contiguous ranges, each range yields a partial (running max m, sum l, unnormalised acc), and the
    partials are merged with weights ``exp(m_s - max_s m_s)``; empty ranges contribute nothing.
    This is the decomposition the HIP kernel uses across workgroups; softmax is invariant to it, so
    it must equal ``attention_fp32`` up to float32 rounding for every split count."""
    rep = q.shape[0] // k.shape[0]
    kr, vr = k.repeat_interleave(rep, 0), v.repeat_interleave(rep, 0)
    L = k.shape[1]
    parts = []
    for sidx in range(splits):
        a, b = (L * sidx) // splits, (L * (sidx + 1)) // splits
        if a == b:
            continue
        s = torch.einsum("hd,hld->hl", q, kr[:, a:b]) * scale
        m = s.amax(-1, keepdim=True)
        e = torch.exp(s - m)
        parts.append((m, e.sum(-1, keepdim=True), torch.einsum("hl,hld->hd", e, vr[:, a:b])))
    M = torch.stack([p[0] for p in parts]).amax(0)
    lsum = sum(p[1] * torch.exp(p[0] - M) for p in parts)
    acc = sum(p[2] * torch.exp(p[0] - M) for p in parts)
    return acc / lsum


def prefill(W, ids, cos, sin, max_seq, position=0, k_cache=None, v_cache=None, causal=True):
    """Batched form of ``decode_step(..., numerics="fp32")`` run once per token: the tokens ``ids``
    (list or 1-D tensor) at positions ``position .. position + len(ids) - 1`` go through the model
    together (fp32 matrix products over all rows, causal fp32 softmax attention), their K/V rows
    are written to the bf16 caches ``[L, Hkv, max_seq, D]`` (new ones if not given; positions before
    ``position`` must already hold earlier tokens), and the logits of the last token are returned.
    This is the arithmetic of a prefill that keeps the reference kernel's fp32 activations
    (/root/reference/megakernel.cu), the work Transformers' prefill does at /root/reference/model.py:72-73.
    ``causal=False`` lets every row see every key of the prompt (a planted mistake for tests).
    Returns (fp32 logits [V], k_cache, v_cache)."""
    s = W.shape
    D, eps = s.head_dim, s.eps
    scale = D ** -0.5
    ids = torch.as_tensor(ids, dtype=torch.long).reshape(-1)
    P = ids.numel()
    if k_cache is None:
        k_cache = torch.zeros(s.layers, s.kv_heads, max_seq, D, dtype=torch.bfloat16)
        v_cache = torch.zeros_like(k_cache)
    pos = torch.arange(position, position + P)
    half = D // 2
    c = cos[pos].float()[:, None, :half]
    sn = sin[pos].float()[:, None, :half]
    T = position + P
    causal = torch.arange(T)[None, :] <= (pos[:, None] if causal else T)  # [P, T]: key t visible to row p
    rep = s.q_heads // s.kv_heads
    x = W.embed[ids].float().clone()

    def rms(t, w):
        return t * torch.rsqrt((t * t).mean(-1, keepdim=True) + eps) * w

    def nr(t, w):
        t = rms(t, w)
        a, b = t[..., :half], t[..., half:]
        return torch.cat((a * c - b * sn, b * c + a * sn), -1)

    for li, lw in enumerate(W.layers):
        h = rms(x, lw["input_layernorm"])
        q = (h @ lw["q_proj"].T).view(P, s.q_heads, D)
        k = (h @ lw["k_proj"].T).view(P, s.kv_heads, D)
        v = (h @ lw["v_proj"].T).view(P, s.kv_heads, D)
        q, k = nr(q, lw["q_norm"]), nr(k, lw["k_norm"])
        k_cache[li, :, position:T] = k.transpose(0, 1).to(torch.bfloat16)
        v_cache[li, :, position:T] = v.transpose(0, 1).to(torch.bfloat16)
        kk = k_cache[li, :, :T].float().repeat_interleave(rep, 0)  # [Hq, T, D]
        vv = v_cache[li, :, :T].float().repeat_interleave(rep, 0)
        sc = (q.transpose(0, 1) @ kk.transpose(1, 2)) * scale      # [Hq, P, T]
        sc = sc.masked_fill(~causal[None], -math.inf)
        attn = (torch.softmax(sc, -1) @ vv).transpose(0, 1).reshape(P, -1)
        x = x + attn @ lw["o_proj"].T
        h2 = rms(x, lw["post_attention_layernorm"])
        g, u = h2 @ lw["gate_proj"].T, h2 @ lw["up_proj"].T
        x = x + (g / (1 + torch.exp(-g)) * u) @ lw["down_proj"].T
    hfin = rms(x[-1], W.final_norm)
    return W.embed @ hfin, k_cache, v_cache

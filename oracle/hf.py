"""Hugging Face Transformers on CPU: the reference path's own arithmetic. TEST INFRASTRUCTURE ONLY.

The reference drives Transformers for prefill and for its comparison decode
(``/root/reference/model.py:23-27`` load, ``:72-73`` prefill, ``:79-87`` cache copy, ``:159-172``
HF greedy decode). The algorithm therefore lives in the third-party dependency
``transformers`` (pinned here: 5.15.0, with torch 2.10.0), which is installed in this image and on
the GPU box; ``Qwen3ForCausalLM`` is at ``transformers/models/qwen3/modeling_qwen3.py:431-507``.

The Hub checkpoint is unreachable offline, so the model is built from ``Qwen3Config`` with a seeded
random init (``torch.manual_seed(0)``, normal std 0.02, norm weights 1.0, tied embeddings,
rope_theta 1e6) and cast with ``.to(torch.bfloat16)``. That cast also turns the rotary
``inv_freq`` buffer into bf16, which changes every RoPE angle; ``rope_tables`` therefore takes the
tables from the model's own rotary module instead of recomputing them in fp32 the way
``/root/reference/model.py:47-53`` does.
"""

import os
import time

import torch

from .spec import SHAPES, LAYER_WEIGHT_ORDER, WEIGHT_SEED, PROMPT_SEED, INIT_STD


def make_config(shape_name, max_positions=4096):
    from transformers import Qwen3Config
    s = SHAPES[shape_name]
    return Qwen3Config(
        hidden_size=s.hidden, intermediate_size=s.intermediate, num_hidden_layers=s.layers,
        num_attention_heads=s.q_heads, num_key_value_heads=s.kv_heads, head_dim=s.head_dim,
        vocab_size=s.vocab, tie_word_embeddings=True, rms_norm_eps=s.eps,
        rope_parameters={"rope_type": "default", "rope_theta": s.rope_theta},
        max_position_embeddings=max_positions, initializer_range=INIT_STD,
    )


def build_model(shape_name, seed=WEIGHT_SEED, max_positions=4096):
    """Seeded random-init bf16 Qwen3ForCausalLM on CPU, in eval mode."""
    from transformers import Qwen3ForCausalLM
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(make_config(shape_name, max_positions))
    return model.to(torch.bfloat16).eval()


def prompt_ids(n, vocab, seed=PROMPT_SEED):
    """Prompt token ids uniform over the vocabulary (``torch.randint`` with its own generator)."""
    return torch.randint(0, vocab, (1, n), generator=torch.Generator().manual_seed(seed))


def layer_weights(model):
    """The 11-per-layer flat list in the reference's order (``/root/reference/model.py:30-44``)."""
    out = []
    for layer in model.model.layers:
        a, m = layer.self_attn, layer.mlp
        mods = {
            "input_layernorm": layer.input_layernorm.weight, "q_proj": a.q_proj.weight,
            "k_proj": a.k_proj.weight, "v_proj": a.v_proj.weight, "q_norm": a.q_norm.weight,
            "k_norm": a.k_norm.weight, "o_proj": a.o_proj.weight,
            "post_attention_layernorm": layer.post_attention_layernorm.weight,
            "gate_proj": m.gate_proj.weight, "up_proj": m.up_proj.weight, "down_proj": m.down_proj.weight,
        }
        out.extend(mods[k].detach() for k in LAYER_WEIGHT_ORDER)
    return out


def rope_tables(model, max_seq_len):
    """bf16 cos/sin tables ``[max_seq_len, head_dim]`` exactly as the model's rotary module makes them
    (``modeling_qwen3.py:126-137``)."""
    x = torch.zeros(1, 1, dtype=torch.bfloat16)
    pos = torch.arange(max_seq_len).unsqueeze(0)
    with torch.inference_mode():
        cos, sin = model.model.rotary_emb(x, pos)
    return cos[0].contiguous(), sin[0].contiguous()


def prefill(model, ids):
    """Run the Transformers prefill (``/root/reference/model.py:72-73``); returns (bf16 logits of the
    last position, DynamicCache)."""
    with torch.inference_mode():
        out = model(ids, use_cache=True)
    return out.logits[0, -1].clone(), out.past_key_values


def cache_to_kernel_layout(hf_cache, num_layers, kv_heads, max_seq_len, head_dim):
    """Copy a DynamicCache into the reference's kernel layout ``[L, Hkv, max_seq, D]`` bf16
    (``/root/reference/model.py:79-87``). Unwritten positions are zero."""
    P = hf_cache.layers[0].keys.shape[2]
    k = torch.zeros(num_layers, kv_heads, max_seq_len, head_dim, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    for layer in range(num_layers):
        k[layer, :, :P] = hf_cache.layers[layer].keys[0]
        v[layer, :, :P] = hf_cache.layers[layer].values[0]
    return k, v


def decode_step(model, token, hf_cache):
    """One Transformers decode step (``/root/reference/model.py:163-172``): bf16 logits [V]."""
    with torch.inference_mode():
        out = model(torch.tensor([[int(token)]]), past_key_values=hf_cache, use_cache=True)
    return out.logits[0, -1].clone(), out.past_key_values


def greedy_reference(model, ids, steps):
    """Prefill then ``steps`` greedy decode steps. Returns dict with the fed tokens, the bf16 logits
    of every decode step, per-step seconds, and the final cache.

    Step t feeds ``tokens[t]`` at position ``P + t`` and yields ``logits[t]``; ``tokens[0]`` is the
    argmax of the prefill logits, ``tokens[t+1]`` the argmax of ``logits[t]`` (first index on ties,
    as ``torch.argmax`` of ``.float()`` logits in ``/root/reference/model.py:97``)."""
    last, cache = prefill(model, ids)
    tokens, logits, secs = [], [], []
    tok = int(last.float().argmax())
    for _ in range(steps):
        tokens.append(tok)
        t0 = time.perf_counter()
        lg, cache = decode_step(model, tok, cache)
        secs.append(time.perf_counter() - t0)
        logits.append(lg)
        tok = int(lg.float().argmax())
    return {"tokens": tokens, "logits": torch.stack(logits) if logits else None, "seconds": secs,
            "cache": cache, "prefill_logits": last}


def cpu_threads():
    """Threads the CPU baseline uses: every core this process may run on."""
    return len(os.sched_getaffinity(0))


def float64_decode_step(model, k_cache, v_cache, token, position, cos, sin):
    """Transformers' own decode step run in float64, with the kernel's inputs: the bf16 cache
    ``[L, Hkv, max_seq, D]`` (positions ``[0, position)``), the bf16 RoPE tables ``cos``/``sin``
    ``[max_seq, D]`` and the new K/V rounded to bf16 as the kernel stores them before attending
    (the reference kernel writes K/V to the cache and attention reads them back,
    ``/root/reference/megakernel.cu:613-619``, ``:270-309``). Returns float64 logits [V].

    This is the independent pin of the float32 restatement (``restate.decode_step(...,
    numerics="fp32")``): same inputs, Transformers' code (``modeling_qwen3.py:241-323``, eager
    attention with a float32 softmax) at higher precision, so the two may differ only by float32
    rounding. Does not modify ``model`` or the caches."""
    import copy

    from transformers import DynamicCache

    m = copy.deepcopy(model).double()
    m.config._attn_implementation = "eager"
    m.model.rotary_emb.forward = lambda x, pos: (cos[pos].double(), sin[pos].double())
    cache = DynamicCache()
    for layer in range(k_cache.shape[0]):
        cache.update(k_cache[layer:layer + 1, :, :position].double(), v_cache[layer:layer + 1, :, :position].double(),
                     layer)
    for cl in cache.layers:
        upd = cl.update
        cl.update = (lambda k, v, *a, upd=upd, **kw:
                     upd(k.to(torch.bfloat16).double(), v.to(torch.bfloat16).double(), *a, **kw))
    with torch.inference_mode():
        out = m(torch.tensor([[int(token)]]), past_key_values=cache, use_cache=True,
                position_ids=torch.tensor([[int(position)]]))
    return out.logits[0, -1].clone()

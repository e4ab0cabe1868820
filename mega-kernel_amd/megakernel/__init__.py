"""MI355X batch-1 decode mega-kernel: Python surface.

The operator is the compiled PyTorch-ROCm extension ``megakernel_extension`` (the reference's
extension name, ``/root/reference/model.py:14-20``), built in-tree by ``megakernel.build``. Its
``decode`` has the reference's signature (``/root/reference/pytorch_binding.cu:36-48``):

    kernel = megakernel.load()
    logits = kernel.decode(token, embed, lm_head, final_norm, layer_weights, cos, sin,
                           k_cache, v_cache, position, max_seq_len)

``load()`` never falls back to anything: if the extension is not built it raises.
Helpers here prepare the operator's inputs the way the reference driver does
(``/root/reference/model.py:30-53``, ``:79-87``).
"""

import importlib.util
import os
import sys

from . import build as _build

EXT_NAME = _build.EXT_NAME
HEAD_DIM = 128
KV_HEADS = 8
_module = None


def load():
    """Return the built ``megakernel_extension`` module. Raises ImportError when it is missing."""
    global _module
    if _module is not None:
        return _module
    path = _build.ext_path()
    if not os.path.exists(path) or not os.path.exists(_build.LIB):
        raise ImportError(
            f"megakernel: the HIP extension is not built ({path}); run `python -m megakernel.build` "
            "from mega-kernel_amd/ or __graft_entry__.build()")
    import torch  # noqa: F401  (loads torch's HIP runtime before the extension)
    spec = importlib.util.spec_from_file_location(EXT_NAME, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules.setdefault(EXT_NAME, mod)
    _module = mod
    return mod


def layer_weight_list(model):
    """The flat 11-tensors-per-layer list in the reference's order (``/root/reference/model.py:30-44``)
    from a Transformers ``Qwen3ForCausalLM``."""
    out = []
    for layer in model.model.layers:
        a, m = layer.self_attn, layer.mlp
        out.extend([layer.input_layernorm.weight, a.q_proj.weight, a.k_proj.weight, a.v_proj.weight,
                    a.q_norm.weight, a.k_norm.weight, a.o_proj.weight, layer.post_attention_layernorm.weight,
                    m.gate_proj.weight, m.up_proj.weight, m.down_proj.weight])
    return [t.detach() for t in out]


def rope_tables(model, max_seq_len, device=None):
    """bf16 cos/sin ``[max_seq_len, 128]`` from the model's own rotary module, so decode positions use
    exactly the angles the Transformers prefill used. (The reference recomputes them in fp32,
    ``/root/reference/model.py:47-53``; after ``model.to(bfloat16)`` Transformers' ``inv_freq`` is
    bf16, so that recomputation would not match the prefilled keys.)"""
    import torch
    ref = next(model.parameters())
    x = torch.zeros(1, 1, dtype=torch.bfloat16, device=ref.device)
    pos = torch.arange(max_seq_len, device=ref.device).unsqueeze(0)
    with torch.inference_mode():
        cos, sin = model.model.rotary_emb(x, pos)
    cos, sin = cos[0].contiguous(), sin[0].contiguous()
    if device is not None:
        cos, sin = cos.to(device), sin.to(device)
    return cos, sin


def empty_cache(num_layers, max_seq_len, device):
    """Zeroed K and V caches ``[num_layers, 8, max_seq_len, 128]`` bf16 (the reference's layout)."""
    import torch
    shape = (num_layers, KV_HEADS, max_seq_len, HEAD_DIM)
    return (torch.zeros(shape, dtype=torch.bfloat16, device=device),
            torch.zeros(shape, dtype=torch.bfloat16, device=device))


def copy_prefill_cache(hf_cache, k_cache, v_cache):
    """Copy a Transformers DynamicCache into the kernel cache (``/root/reference/model.py:79-87``).
    Returns the number of prefilled positions."""
    n = 0
    for layer in range(k_cache.shape[0]):
        k = hf_cache.layers[layer].keys[0]
        v = hf_cache.layers[layer].values[0]
        n = k.shape[1]
        k_cache[layer, :, :n] = k.to(k_cache.device)
        v_cache[layer, :, :n] = v.to(v_cache.device)
    return n

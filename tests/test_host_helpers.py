"""CPU tests of the product's own host helpers (``megakernel``), which prepare the operator's inputs
the way the reference driver does (/root/reference/model.py:30-53, :79-87). Each is checked against
the oracle's independent version or against Transformers' own tensors."""
import torch

import megakernel
from oracle import hf
from oracle.spec import LAYER_WEIGHT_ORDER, SHAPES


def _tiny():
    return hf.build_model("tiny", max_positions=256)


def test_rope_tables_equal_the_models_rotary_embedding():
    """``megakernel.rope_tables`` gives, for every position, the cos/sin the model's attention uses
    (``modeling_qwen3.py:126-137`` via ``rotary_emb``), i.e. the angles the Transformers prefill
    rotated its keys with; bf16 ``[max_seq, head_dim]``. Also the closed form: with the model's bf16
    ``inv_freq``, cos/sin of ``p * inv_freq`` duplicated over both halves."""
    model = _tiny()
    s = SHAPES["tiny"]
    cos, sin = megakernel.rope_tables(model, 200)
    assert cos.dtype == torch.bfloat16 and cos.shape == (200, s.head_dim) and sin.shape == (200, s.head_dim)
    ocos, osin = hf.rope_tables(model, 200)
    assert torch.equal(cos, ocos) and torch.equal(sin, osin)
    inv = model.model.rotary_emb.inv_freq.float()
    ang = torch.arange(200, dtype=torch.float32)[:, None] * inv[None, :]
    want_c = torch.cat((ang.cos(), ang.cos()), -1)
    want_s = torch.cat((ang.sin(), ang.sin()), -1)
    assert (cos.float() - want_c).abs().max().item() <= 2 ** -8
    assert (sin.float() - want_s).abs().max().item() <= 2 ** -8


def test_copy_prefill_cache_places_rows_in_the_kernel_layout():
    """``megakernel.copy_prefill_cache`` moves a Transformers DynamicCache (``[1, Hkv, P, D]`` per
    layer) into the kernel's ``[L, Hkv, max_seq, D]`` cache: row p of head h of layer l lands at
    ``[l, h, p]``, positions past the prompt stay untouched, and it returns P."""
    model = _tiny()
    s = SHAPES["tiny"]
    P, max_seq = 13, 40
    ids = hf.prompt_ids(P, s.vocab)
    _, cache = hf.prefill(model, ids)
    k = torch.full((s.layers, s.kv_heads, max_seq, s.head_dim), 7.0, dtype=torch.bfloat16)
    v = torch.full_like(k, 7.0)
    assert megakernel.copy_prefill_cache(cache, k, v) == P
    for layer in range(s.layers):
        assert torch.equal(k[layer, :, :P], cache.layers[layer].keys[0])
        assert torch.equal(v[layer, :, :P], cache.layers[layer].values[0])
    assert (k[:, :, P:] == 7.0).all() and (v[:, :, P:] == 7.0).all()
    ko, vo = hf.cache_to_kernel_layout(cache, s.layers, s.kv_heads, max_seq, s.head_dim)
    assert torch.equal(k[:, :, :P], ko[:, :, :P]) and torch.equal(v[:, :, :P], vo[:, :, :P])


def test_layer_weight_list_is_the_reference_order():
    """``megakernel.layer_weight_list``: 11 tensors per layer in the order of
    /root/reference/model.py:30-44 (the ``LayerWeights`` field order), the same tensors the oracle
    names."""
    model = _tiny()
    got = megakernel.layer_weight_list(model)
    want = hf.layer_weights(model)
    assert len(got) == len(LAYER_WEIGHT_ORDER) * SHAPES["tiny"].layers
    for a, b in zip(got, want):
        assert a.data_ptr() == b.data_ptr()


def test_bench_bytes_per_token_matches_the_pinned_count():
    """bench.py's algorithmic bytes per step equal the oracle's count, which test_oracle pins against
    the Transformers model's own parameter sizes."""
    import bench
    for name in ("qwen3-0.6b", "qwen3-1.7b"):
        s = SHAPES[name]
        for ctx in (1, 33, 288, 3840):
            assert bench.bytes_per_token(s.hidden, s.intermediate, s.layers, s.vocab, ctx) == s.bytes_per_token(ctx)

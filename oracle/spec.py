"""Model shapes and the synthetic-input protocol shared by the oracle, tests and bench.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference hard-codes Qwen3-0.6B (``/root/reference/config.cuh:9-18``); the 1.7B shape and the
tiny shape are the extra configurations the parity tests run. ``LAYER_WEIGHT_ORDER`` is the order in
which the reference flattens 11 tensors per layer (``/root/reference/model.py:30-44``), which is also
the field order of its ``LayerWeights`` table (``/root/reference/config.cuh:77-89``).
"""

from dataclasses import dataclass

LAYER_WEIGHT_ORDER = (
    "input_layernorm",          # [H]
    "q_proj",                   # [Hq*D, H]
    "k_proj",                   # [Hkv*D, H]
    "v_proj",                   # [Hkv*D, H]
    "q_norm",                   # [D]
    "k_norm",                   # [D]
    "o_proj",                   # [H, Hq*D]
    "post_attention_layernorm", # [H]
    "gate_proj",                # [I, H]
    "up_proj",                  # [I, H]
    "down_proj",                # [H, I]
)


@dataclass(frozen=True)
class Shape:
    name: str
    hidden: int
    intermediate: int
    layers: int
    q_heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def q_size(self):
        return self.q_heads * self.head_dim

    @property
    def kv_size(self):
        return self.kv_heads * self.head_dim

    def weight_bytes_per_token(self):
        """Algorithmic weight bytes one decode step must read (bf16): every layer weight, the
        full tied LM head, one embedding row and the final norm."""
        H, I, D = self.hidden, self.intermediate, self.head_dim
        per_layer = (self.q_size * H + 2 * self.kv_size * H + H * self.q_size + 3 * I * H) * 2
        per_layer += (2 * H + 2 * D) * 2
        return self.layers * per_layer + self.vocab * H * 2 + H * 2 + H * 2

    def kv_bytes_per_position(self):
        """K and V bytes per cached position, all layers (bf16)."""
        return self.layers * self.kv_heads * self.head_dim * 2 * 2

    def bytes_per_token(self, ctx):
        """B(ctx) = W + kv_read(ctx) + kv_write + cos/sin row."""
        return (self.weight_bytes_per_token() + self.kv_bytes_per_position() * ctx
                + self.kv_bytes_per_position() + 2 * self.head_dim * 2)


SHAPES = {
    "qwen3-0.6b": Shape("qwen3-0.6b", 1024, 3072, 28, 16, 8, 128, 151936),
    "qwen3-1.7b": Shape("qwen3-1.7b", 2048, 6144, 28, 16, 8, 128, 151936),
    # small enough for pure-CPU fixture tests
    "tiny": Shape("tiny", 64, 192, 2, 4, 2, 16, 512),
    # the kernel's fixed head geometry (16 q / 8 kv heads of 128) with few layers and a small vocab
    "mini": Shape("mini", 1024, 3072, 2, 16, 8, 128, 4096),
    "mini-1.7b": Shape("mini-1.7b", 2048, 6144, 2, 16, 8, 128, 4096),
}

WEIGHT_SEED = 0   # torch.manual_seed before constructing the model
PROMPT_SEED = 1   # torch.Generator seed for prompt ids
INIT_STD = 0.02

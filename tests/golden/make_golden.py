"""Write the committed golden fixtures for the CPU oracle tests.

The reference (tejeshbhalla/mega-kernel) has no tests, fixtures or known-answer vectors for its
decode path; its arithmetic lives in Hugging Face Transformers, which its driver runs for prefill and
for its comparison decode (/root/reference/model.py:72-73, :159-172). This script runs that
third-party path -- Transformers ``Qwen3ForCausalLM`` on the CPU, the version installed in this
image -- on a tiny seeded random-init model and stores inputs and outputs:

  weights (bf16: embedding, final norm, 11 tensors per layer in the reference's order
  /root/reference/model.py:30-44), prompt ids, the prefill K/V in the kernel cache layout
  [L, Hkv, max_seq, D] (/root/reference/model.py:79-87), the bf16 RoPE tables, the greedy tokens
  fed at each decode step and the bf16 logits Transformers returned for each step.

    python tests/golden/make_golden.py            # rewrites tests/golden/tiny_decode.safetensors
"""
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import hf  # noqa: E402
from oracle.spec import SHAPES  # noqa: E402

SHAPE = "tiny"
PROMPT = 12
STEPS = 8
MAX_SEQ = 32


def main():
    torch.set_num_threads(1)
    s = SHAPES[SHAPE]
    model = hf.build_model(SHAPE, max_positions=MAX_SEQ)
    ids = hf.prompt_ids(PROMPT, s.vocab)
    ref = hf.greedy_reference(model, ids, STEPS)
    _, cache = hf.prefill(model, ids)
    kc, vc = hf.cache_to_kernel_layout(cache, s.layers, s.kv_heads, MAX_SEQ, s.head_dim)
    cos, sin = hf.rope_tables(model, MAX_SEQ)
    t = {
        "embed": model.model.embed_tokens.weight.detach().contiguous(),
        "final_norm": model.model.norm.weight.detach().contiguous(),
        "prompt_ids": ids[0].to(torch.int64).contiguous(),
        "k_cache": kc.contiguous(), "v_cache": vc.contiguous(),
        "cos": cos.contiguous(), "sin": sin.contiguous(),
        "tokens": torch.tensor(ref["tokens"], dtype=torch.int64),
        "logits": ref["logits"].contiguous(),
        "prefill_logits": ref["prefill_logits"].contiguous(),
    }
    for i, w in enumerate(hf.layer_weights(model)):
        t[f"layer_weights.{i:03d}"] = w.contiguous()
    meta = {"shape": SHAPE, "prompt": str(PROMPT), "steps": str(STEPS), "max_seq": str(MAX_SEQ),
            "generator": "transformers " + __import__("transformers").__version__ + ", torch " + torch.__version__,
            "cpu_threads": "1"}
    out = os.path.join(HERE, "tiny_decode.safetensors")
    save_file(t, out, metadata=meta)
    print(json.dumps({"wrote": out, "bytes": os.path.getsize(out), **meta}))


if __name__ == "__main__":
    main()

"""Greedy decoding driver: the reference's Python surface on the MI355X decode kernel.

Mirrors ``/root/reference/model.py`` step for step:
  * build the model (``:23-27``). The Hub checkpoint is unreachable offline, so this builds a seeded
    random-init Qwen3 of the requested shape (normal std 0.02, norms 1, tied embeddings,
    rope_theta 1e6) on the CPU and casts it to bf16. The Transformers prefill runs on the CPU
    (torch's bf16 batched products on this GPU are avoided); its weights, RoPE tables and K/V are
    then copied to the GPU;
  * flatten the 11 weights per layer (``:30-44``) and build the RoPE tables (``:47-53``, taken from
    the model's own rotary module, see ``megakernel.rope_tables``);
  * prefill with Transformers (``:72-73``) and copy its K/V into the ``[L, 8, max_seq, 128]`` cache
    (``:79-87``);
  * greedy loop calling the same ``decode`` entry point (``:95-127``), timed with device events.
    The fused device argmax (``decode_greedy``) replaces the separate ``argmax().item()`` per token;
    the host reads each token back only to feed the next call, as the reference does.
  * ``--device-loop``: the same greedy generation as one ``decode_steps`` call, which feeds each
    step's argmax to the next launch on the device; the host reads the tokens once at the end.
  * ``--native-prefill``: the prompt goes through the batched prefill kernel (``prefill``: all
    prompt tokens at once on the matrix cores, writing the ``[L, 8, max_seq, 128]`` cache
    directly) instead of the Transformers prefill and cache copy.

    python mega-kernel_amd/model.py [--shape qwen3-0.6b] [--prompt 32] [--max-seq 512] [--new 64]
                                    [--device-loop] [--native-prefill]
"""
import argparse
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

SHAPES = {  # hidden, intermediate (28 layers, 16 q / 8 kv heads of 128, vocab 151936)
    "qwen3-0.6b": (1024, 3072),
    "qwen3-1.7b": (2048, 6144),
}


def build_model(shape, max_positions, seed=0):
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    hidden, inter = SHAPES[shape]
    cfg = Qwen3Config(hidden_size=hidden, intermediate_size=inter, num_hidden_layers=28, num_attention_heads=16,
                      num_key_value_heads=8, head_dim=128, vocab_size=151936, tie_word_embeddings=True,
                      rms_norm_eps=1e-6, rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                      max_position_embeddings=max_positions, initializer_range=0.02)
    torch.manual_seed(seed)
    return Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()


def run(argv=None, keep_prefill_cache=False):
    """Runs the driver and returns what it did: the generated tokens (the prefill's greedy token
    first), the prompt length, the device status after the loop, ms per token, and, with
    ``keep_prefill_cache``, a copy of the K/V cache as the prefill left it together with the decode
    operator's other inputs (so a caller can replay the decode from the same state)."""
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", default="qwen3-0.6b", choices=sorted(SHAPES))
    ap.add_argument("--prompt", type=int, default=32, help="random prompt length (token ids, seed 1)")
    ap.add_argument("--max-seq", type=int, default=512)
    ap.add_argument("--new", type=int, default=64, help="tokens to generate")
    ap.add_argument("--device-loop", action="store_true", help="generate with one decode_steps call")
    ap.add_argument("--native-prefill", action="store_true",
                    help="fill the cache with the batched prefill kernel (prefill) instead of the Transformers "
                         "prefill and cache copy")
    a = ap.parse_args(argv)
    import torch
    import megakernel

    kernel = megakernel.load()  # the HIP operator; raises if it is not built
    dev = torch.device("cuda:0")
    model = build_model(a.shape, max(4096, a.max_seq))
    ids = torch.randint(0, 151936, (1, a.prompt), generator=torch.Generator().manual_seed(1))
    layer_weights = [t.to(dev) for t in megakernel.layer_weight_list(model)]
    embed = model.model.embed_tokens.weight.detach().to(dev)
    final_norm = model.model.norm.weight.detach().to(dev)
    cos, sin = megakernel.rope_tables(model, a.max_seq, dev)

    k_cache, v_cache = megakernel.empty_cache(len(model.model.layers), a.max_seq, dev)
    if a.native_prefill:
        prompt = ids[0].to(device=dev, dtype=torch.int32)
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p0.record()
        _, first = kernel.prefill(prompt, embed, embed, final_norm, layer_weights, cos, sin, k_cache, v_cache, 0,
                                  a.max_seq)
        p1.record()
        position, token = a.prompt, int(first.item())
        print(f"prefill: {a.prompt} tokens in {p0.elapsed_time(p1):.2f} ms (batched prefill kernel)")
    else:
        with torch.inference_mode():
            out = model(ids, use_cache=True)
        position = megakernel.copy_prefill_cache(out.past_key_values, k_cache, v_cache)
        token = int(out.logits[0, -1].float().argmax())
    result = {"prompt": position, "first_token": token}
    if keep_prefill_cache:
        result["prefill_cache"] = (k_cache.clone(), v_cache.clone())
        result["inputs"] = {"embed": embed, "final_norm": final_norm, "layer_weights": layer_weights, "cos": cos,
                            "sin": sin, "max_seq": a.max_seq}

    generated = [token]
    steps = min(a.new, a.max_seq - position)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    if a.device_loop and steps > 1:
        tokens = torch.zeros(steps, dtype=torch.int32, device=dev)
        tokens[0] = token
        kernel.decode_steps(tokens, steps - 1, True, embed, embed, final_norm, layer_weights, cos, sin, k_cache,
                            v_cache, position, a.max_seq)
    else:
        for _ in range(steps - 1):
            _, tok = kernel.decode_greedy(token, embed, embed, final_norm, layer_weights, cos, sin, k_cache,
                                          v_cache, position, a.max_seq)
            token = int(tok.item())
            generated.append(token)
            position += 1
    end.record()
    end.synchronize()
    wall = time.perf_counter() - t0
    if a.device_loop and steps > 1:
        generated = tokens.tolist()
    n = max(steps - 1, 1)
    result.update(generated=generated, status=kernel.status(), ms_per_token=start.elapsed_time(end) / n)
    print(f"generated {len(generated)} tokens: {generated[:16]}{' ...' if len(generated) > 16 else ''}")
    print(f"decode: {result['ms_per_token']:.3f} ms/token (device events), {n / wall:.1f} tokens/s wall, "
          f"device status {result['status']}")
    return result


def main(argv=None):
    """The command line: 0 when the device status is clean and every generated token is valid."""
    r = run(argv)
    return 0 if r["status"] == 0 and all(t >= 0 for t in r["generated"]) else 1


if __name__ == "__main__":
    sys.exit(main())

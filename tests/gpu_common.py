"""Shared pieces of the GPU parity tests: a model session (oracle weights on the CPU, the same bf16
weights on the GPU), the C-ABI library through ctypes, and the statistics the tests assert on.

Only the tests import this module; it needs a GPU for everything but ``stats``."""
import ctypes

import torch

from oracle import hf, restate
from oracle.spec import LAYER_WEIGHT_ORDER, SHAPES

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
        # the product helper, not the oracle's: the kernel's tables come from megakernel.rope_tables
        self.cos, self.sin = megakernel.rope_tables(self.model, max_seq, device=DEV)
        self.cos_cpu, self.sin_cpu = hf.rope_tables(self.model, max_seq)
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

    def decode_steps(self, tokens, n, generate, kd, vd, position):
        return self.kernel.decode_steps(tokens, n, generate, self.embed, self.lm_head, self.final_norm, self.layers,
                                        self.cos, self.sin, kd, vd, position, self.max_seq)

    def oracle_step(self, k_cache, v_cache, token, position):
        """The fp32 restatement of one step on CPU caches (written at ``position``)."""
        logits, _ = restate.decode_step(self.W, k_cache, v_cache, int(token), int(position), self.cos_cpu,
                                        self.sin_cpu, numerics="fp32")
        return logits

    def device_layer_table(self):
        """A device ``mk_layer_weights[L]`` built by hand: per layer the 11 data pointers in the order
        of the struct's fields, which is the reference's 11-per-layer order."""
        ptrs = [t.data_ptr() for t in self.layers]
        assert len(ptrs) == len(LAYER_WEIGHT_ORDER) * self.shape.layers
        return torch.tensor(ptrs, dtype=torch.int64, device=DEV)


class Dims(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                ("num_layers", ctypes.c_int32), ("vocab", ctypes.c_int32)]


def c_library():
    """The C-ABI library (the same file the extension links, so the same per-device state)."""
    from megakernel import build as mkbuild
    lib = ctypes.CDLL(mkbuild.LIB)
    vp = ctypes.c_void_p
    decode_args = [ctypes.POINTER(Dims), ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int,
                   vp, vp, vp]
    for name in ("mk_decode", "mk_decode_noalloc"):
        if hasattr(lib, name):
            f = getattr(lib, name)
            f.restype = ctypes.c_int
            f.argtypes = decode_args
    lib.launch_decode_kernel.restype = ctypes.c_int
    lib.launch_decode_kernel.argtypes = [ctypes.c_int] + [vp] * 18 + [ctypes.c_int] * 3 + [vp]
    return lib


def stream_handle():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def stats(ours, ref):
    """(max-abs difference, cosine similarity) in float64."""
    ours, ref = ours.double(), ref.double()
    cos = torch.nn.functional.cosine_similarity(ours, ref, dim=0).item()
    return (ours - ref).abs().max().item(), cos


def parity_dir():
    """Where the parity tests leave their per-config records: ``$MK_PARITY_DIR``, else
    ``gpurun_out/parity`` under the repository root."""
    import os
    d = os.environ.get("MK_PARITY_DIR") or os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                                       "gpurun_out", "parity")
    os.makedirs(d, exist_ok=True)
    return d


def write_record(name, rec):
    """One parity record as JSON (``<name>.json`` in ``parity_dir()``), with the kernel version and
    the GPU it ran on, so that a summary can be rebuilt from the files alone."""
    import json
    import os
    import megakernel
    out = dict(rec)
    out["kernel_version"] = megakernel.load().version()
    out["device"] = torch.cuda.get_device_name(0) if torch.cuda.is_available() else None
    path = os.path.join(parity_dir(), f"{name}.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    return path

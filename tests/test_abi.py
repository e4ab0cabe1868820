"""Host-side tests of the drop-in boundary: the C-ABI library and the PyTorch operator load, export
what ``include/megakernel_amd.h`` declares, and reject bad arguments before anything is launched
(the reference validates nothing, /root/reference/pytorch_binding.cu:36-129; its errors surface only
from CUDA calls). No GPU is used: every call here returns before the first HIP runtime call."""
import ctypes
import os
import re

import pytest
import torch

from megakernel import build as mkbuild

HEADER = os.path.join(mkbuild.INCLUDE, "megakernel_amd.h")
HIP_SUCCESS, HIP_ERROR_INVALID_VALUE = 0, 1


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(mk_\w+|launch_decode_kernel)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(mkbuild.LIB), "libmegakernel_amd.so is not built (run __graft_entry__.build())"
    return ctypes.CDLL(mkbuild.LIB)


def test_header_declares_the_reference_launcher_and_the_library_exports_everything(lib):
    names = declared_functions()
    assert "launch_decode_kernel" in names and "mk_decode" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in megakernel_amd.h but not exported"


def test_version(lib):
    lib.mk_version.restype = ctypes.c_char_p
    assert lib.mk_version().decode().startswith("megakernel_amd")


def test_trace_bytes(lib):
    lib.mk_trace_bytes.restype = ctypes.c_size_t
    n = lib.mk_trace_bytes()
    assert n > 0 and n % 8 == 0


def test_c_abi_rejects_bad_arguments_before_launch(lib):
    """hipErrorInvalidValue for a null shape, an unsupported shape, a token or position out of range
    and (reference launcher) cache_len != position + 1 -- no device is touched."""
    f = lib.mk_decode
    f.restype = ctypes.c_int
    vp = ctypes.c_void_p
    f.argtypes = [vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, vp]
    dummy = vp(16)

    class Dims(ctypes.Structure):
        _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                    ("num_layers", ctypes.c_int32), ("vocab", ctypes.c_int32)]

    def call(dims, token=1, position=3, max_seq=512, logits=dummy):
        d = ctypes.byref(dims) if dims is not None else None
        return f(d, token, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, position, max_seq, logits, None, None)

    good = Dims(1024, 3072, 28, 151936)
    assert call(None) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 4096, 28, 151936)) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 3072, 0, 151936)) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 3072, 28, 255)) == HIP_ERROR_INVALID_VALUE  # fewer vocabulary rows than workgroups
    assert call(good, token=-1) == HIP_ERROR_INVALID_VALUE
    assert call(good, token=151936) == HIP_ERROR_INVALID_VALUE
    assert call(good, position=512) == HIP_ERROR_INVALID_VALUE
    assert call(good, position=-1) == HIP_ERROR_INVALID_VALUE
    assert call(good, logits=None) == HIP_ERROR_INVALID_VALUE

    g = lib.launch_decode_kernel
    g.restype = ctypes.c_int
    g.argtypes = [ctypes.c_int] + [vp] * 18 + [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
    assert g(1, *([dummy] * 18), 10, 10, 512, None) == HIP_ERROR_INVALID_VALUE  # cache_len must be position + 1

    # the device-side multi-token loop: n >= 1 steps that all fit in the cache, a token array
    s = lib.mk_decode_steps
    s.restype = ctypes.c_int
    s.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int] + [vp] * 8 + [ctypes.c_int, ctypes.c_int, vp, vp]

    def steps(dims=good, tokens=dummy, n=4, position=3, max_seq=512, generate=1):
        d = ctypes.byref(dims) if dims is not None else None
        return s(d, tokens, n, generate, *([dummy] * 8), position, max_seq, dummy, None)

    assert steps(dims=None) == HIP_ERROR_INVALID_VALUE
    assert steps(tokens=None) == HIP_ERROR_INVALID_VALUE
    assert steps(n=0) == HIP_ERROR_INVALID_VALUE
    assert steps(position=509, n=4) == HIP_ERROR_INVALID_VALUE  # the last step would write position 512
    assert steps(position=509, n=4, generate=0) == HIP_ERROR_INVALID_VALUE
    assert steps(Dims(2048, 3072, 28, 151936)) == HIP_ERROR_INVALID_VALUE

    # the paged cache: a block table, a power-of-two page size, at most 2048 table entries
    pg = lib.mk_decode_paged
    pg.restype = ctypes.c_int
    pg.argtypes = [vp, ctypes.c_int] + [vp] * 9 + [ctypes.c_int] * 4 + [vp, vp, vp]

    def paged(table=dummy, num_pages=64, page=16, position=3, max_seq=512, token=1):
        return pg(ctypes.byref(good), token, *([dummy] * 8), table, num_pages, page, position, max_seq, dummy,
                  None, None)

    assert paged(table=None) == HIP_ERROR_INVALID_VALUE
    assert paged(num_pages=0) == HIP_ERROR_INVALID_VALUE
    assert paged(page=24) == HIP_ERROR_INVALID_VALUE
    assert paged(page=8192) == HIP_ERROR_INVALID_VALUE
    assert paged(page=1, max_seq=4096) == HIP_ERROR_INVALID_VALUE  # 4096 table entries > 2048
    assert paged(position=512) == HIP_ERROR_INVALID_VALUE
    assert paged(token=151936) == HIP_ERROR_INVALID_VALUE

    sp = lib.mk_decode_steps_paged
    sp.restype = ctypes.c_int
    sp.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int] + [vp] * 9 + [ctypes.c_int] * 4 + [vp, vp]

    def steps_paged(tokens=dummy, n=4, table=dummy, page=16, position=3, max_seq=512):
        return sp(ctypes.byref(good), tokens, n, 1, *([dummy] * 8), table, 64, page, position, max_seq, dummy, None)

    assert steps_paged(tokens=None) == HIP_ERROR_INVALID_VALUE
    assert steps_paged(n=0) == HIP_ERROR_INVALID_VALUE
    assert steps_paged(table=None) == HIP_ERROR_INVALID_VALUE
    assert steps_paged(page=12) == HIP_ERROR_INVALID_VALUE
    assert steps_paged(position=509) == HIP_ERROR_INVALID_VALUE


# ---------------------------------------------------------------------------------------------
# the PyTorch operator (reference name and signature)
# ---------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def ext():
    import megakernel
    return megakernel.load()


def _args(L=2, V=300, max_seq=16, dtype=torch.bfloat16):
    """A well-formed argument list on the CPU: the 0.6B layer shapes (hidden 1024, intermediate
    3072, 16 q / 8 kv heads of 128) with few layers, a small vocabulary and a short cache."""
    H, I = 1024, 3072
    mk = lambda *s: torch.zeros(*s, dtype=dtype)
    lw = []
    for _ in range(L):
        lw += [mk(H), mk(2048, H), mk(1024, H), mk(1024, H), mk(128), mk(128), mk(H, 2048), mk(H), mk(I, H),
               mk(I, H), mk(H, I)]
    embed = mk(V, H)
    return [5, embed, embed, mk(H), lw, mk(max_seq, 128), mk(max_seq, 128), mk(L, 8, max_seq, 128),
            mk(L, 8, max_seq, 128), 3, max_seq]


def test_operator_exports_reference_entry_point(ext):
    assert callable(ext.decode) and callable(ext.decode_greedy) and callable(ext.decode_steps)
    assert callable(ext.decode_paged) and callable(ext.decode_steps_paged)
    assert ext.version().startswith("megakernel_amd")


def test_operator_requires_gpu_tensors(ext):
    with pytest.raises(RuntimeError, match="GPU tensor"):
        ext.decode(*_args())


def test_check_args_accepts_well_formed_input(ext):
    assert ext.check_args(*_args()) == (1024, 3072, 2, 300)


@pytest.mark.parametrize("mutate, message", [
    (lambda a: a.__setitem__(0, 300), "token_id"),
    (lambda a: a.__setitem__(0, -1), "token_id"),
    (lambda a: a.__setitem__(9, 16), "position"),
    (lambda a: a.__setitem__(9, -1), "position"),
    (lambda a: a.__setitem__(4, a[4][:-1]), "11 tensors per layer"),
    (lambda a: a.__setitem__(1, a[1].float()), "bfloat16"),
    (lambda a: a.__setitem__(7, a[7].transpose(2, 3).contiguous().transpose(2, 3)), "contiguous"),
    (lambda a: a.__setitem__(7, a[7][:, :, :8].contiguous()), "k_cache"),
    (lambda a: a.__setitem__(8, a[7]), "distinct"),
    (lambda a: a.__setitem__(5, a[5][:8].contiguous()), "cos/sin"),
    (lambda a: a[4].__setitem__(1, torch.zeros(2048, 512, dtype=torch.bfloat16)), "q_proj"),
    (lambda a: a.__setitem__(3, torch.zeros(1023, dtype=torch.bfloat16)), "final_norm"),
])
def test_check_args_rejects(ext, mutate, message):
    a = _args()
    mutate(a)
    with pytest.raises(RuntimeError, match=message):
        ext.check_args(*a)


def test_unsupported_shape_is_rejected(ext):
    a = _args()
    for i in range(len(a[4])):
        if a[4][i].dim() == 2 and a[4][i].shape[0] == 3072:
            a[4][i] = torch.zeros(4096, 1024, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="supported"):
        ext.check_args(*a)


def test_noalloc_entry_point_rejects_out_of_limit_arguments_before_launch(lib):
    """``mk_decode_noalloc`` checks its limits (supported shape, layers, vocabulary, position) before
    any HIP call, like ``mk_decode``; ``mk_workspace_bytes`` reports the static array's size."""
    f = lib.mk_decode_noalloc
    f.restype = ctypes.c_int
    vp = ctypes.c_void_p
    f.argtypes = [vp, ctypes.c_int, vp, vp, vp, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, vp]
    dummy = vp(16)

    class Dims(ctypes.Structure):
        _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                    ("num_layers", ctypes.c_int32), ("vocab", ctypes.c_int32)]

    def call(dims, token=1, position=3, max_seq=512):
        return f(ctypes.byref(dims), token, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, position,
                 max_seq, dummy, None, None)

    assert call(Dims(4096, 12288, 28, 151936)) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 3072, 63, 151936)) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 3072, 28, 255)) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 3072, 28, 151936), position=512) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 3072, 28, 151936), token=151936) == HIP_ERROR_INVALID_VALUE
    lib.mk_workspace_bytes.restype = ctypes.c_size_t
    assert 1 << 20 <= lib.mk_workspace_bytes() <= 2 << 20


def test_prefill_entry_point_rejects_bad_arguments_before_launch(lib):
    """``mk_prefill`` validates shape, token count, positions and the workspace size and alignment
    before any HIP call; ``mk_prefill_workspace_bytes`` grows with the token count."""
    vp, i32 = ctypes.c_void_p, ctypes.c_int

    class Dims(ctypes.Structure):
        _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                    ("num_layers", ctypes.c_int32), ("vocab", ctypes.c_int32)]

    ws = lib.mk_prefill_workspace_bytes
    ws.restype = ctypes.c_size_t
    ws.argtypes = [ctypes.POINTER(Dims), i32]
    good = Dims(1024, 3072, 28, 151936)
    n1, n2 = ws(ctypes.byref(good), 32), ws(ctypes.byref(good), 3584)
    assert 0 < n1 < n2 and n1 % 256 == 0
    assert ws(ctypes.byref(good), 0) == 0

    f = lib.mk_prefill
    f.restype = i32
    f.argtypes = [ctypes.POINTER(Dims), vp, i32, i32] + [vp] * 8 + [i32, vp, vp, vp, ctypes.c_size_t, vp]
    d = vp(256)

    def call(dims=good, n=32, position=0, max_seq=512, workspace=d, nbytes=None):
        nb = ws(ctypes.byref(dims), n) if nbytes is None else nbytes
        return f(ctypes.byref(dims), d, n, position, *([d] * 8), max_seq, d, None, workspace, nb, None)

    assert call(Dims(1024, 4096, 28, 151936)) == HIP_ERROR_INVALID_VALUE
    assert call(n=0) == HIP_ERROR_INVALID_VALUE
    assert call(position=-1) == HIP_ERROR_INVALID_VALUE
    assert call(position=500, n=13) == HIP_ERROR_INVALID_VALUE  # past max_seq_len
    assert call(nbytes=n1 - 1) == HIP_ERROR_INVALID_VALUE
    assert call(workspace=vp(256 + 16)) == HIP_ERROR_INVALID_VALUE  # not 256-byte aligned
    assert call(workspace=None) == HIP_ERROR_INVALID_VALUE



def test_paged_prefill_entry_point_rejects_bad_arguments_before_launch(lib):
    """``mk_prefill_paged`` checks the block table, page count and page size (a power of two up to
    4096, at most 2048 table entries for max_seq_len) before any HIP call, then everything
    ``mk_prefill`` checks."""
    vp, i32 = ctypes.c_void_p, ctypes.c_int

    class Dims(ctypes.Structure):
        _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                    ("num_layers", ctypes.c_int32), ("vocab", ctypes.c_int32)]

    ws = lib.mk_prefill_workspace_bytes
    ws.restype = ctypes.c_size_t
    ws.argtypes = [ctypes.POINTER(Dims), i32]
    good = Dims(1024, 3072, 28, 151936)
    f = lib.mk_prefill_paged
    f.restype = i32
    f.argtypes = [ctypes.POINTER(Dims), vp, i32, i32] + [vp] * 8 + [vp, i32, i32, i32, vp, vp, vp, ctypes.c_size_t, vp]
    d = vp(256)

    def call(table=d, num_pages=64, page_size=16, n=32, position=0, max_seq=512, nbytes=None):
        nb = ws(ctypes.byref(good), n) if nbytes is None else nbytes
        return f(ctypes.byref(good), d, n, position, *([d] * 8), table, num_pages, page_size, max_seq, d, None, d,
                 nb, None)

    assert call(table=None) == HIP_ERROR_INVALID_VALUE
    assert call(num_pages=0) == HIP_ERROR_INVALID_VALUE
    assert call(page_size=24) == HIP_ERROR_INVALID_VALUE   # not a power of two
    assert call(page_size=8192) == HIP_ERROR_INVALID_VALUE
    assert call(page_size=1, max_seq=4096) == HIP_ERROR_INVALID_VALUE  # 4096 table entries
    assert call(position=500, n=13) == HIP_ERROR_INVALID_VALUE  # past max_seq_len
    assert call(nbytes=1024) == HIP_ERROR_INVALID_VALUE

def test_batch_entry_point_rejects_bad_arguments_before_launch(lib):
    """``mk_decode_batch`` checks the batch size (1..64), shape, vocabulary (a multiple of 16: the LM
    head's skinny product takes 16 rows per workgroup), workspace size and alignment before any HIP
    call; ``mk_decode_batch_workspace_bytes`` is 0 for an unsupported batch."""
    vp, i32 = ctypes.c_void_p, ctypes.c_int

    class Dims(ctypes.Structure):
        _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32),
                    ("num_layers", ctypes.c_int32), ("vocab", ctypes.c_int32)]

    ws = lib.mk_decode_batch_workspace_bytes
    ws.restype = ctypes.c_size_t
    ws.argtypes = [ctypes.POINTER(Dims), i32, i32]
    good = Dims(1024, 3072, 28, 151936)
    assert ws(ctypes.byref(good), 0, 512) == 0 and ws(ctypes.byref(good), 65, 512) == 0
    n8 = ws(ctypes.byref(good), 8, 4096)
    assert n8 > ws(ctypes.byref(good), 1, 512) > 0 and n8 % 256 == 0
    assert ws(ctypes.byref(good), 64, 4096) > n8

    f = lib.mk_decode_batch
    f.restype = i32
    f.argtypes = [ctypes.POINTER(Dims), i32, vp, vp] + [vp] * 8 + [i32, vp, vp, vp, ctypes.c_size_t, vp]
    d = vp(256)

    def call(dims=good, batch=4, max_seq=512, workspace=d, nbytes=None):
        nb = ws(ctypes.byref(dims), batch, max_seq) if nbytes is None else nbytes
        return f(ctypes.byref(dims), batch, d, d, *([d] * 8), max_seq, d, None, workspace, nb, None)

    assert call(batch=0) == HIP_ERROR_INVALID_VALUE
    assert call(batch=65) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(2048, 3072, 28, 151936)) == HIP_ERROR_INVALID_VALUE
    assert call(Dims(1024, 3072, 28, 151930)) == HIP_ERROR_INVALID_VALUE  # vocabulary not a multiple of 16
    assert call(nbytes=1024) == HIP_ERROR_INVALID_VALUE
    assert call(workspace=vp(256 + 64)) == HIP_ERROR_INVALID_VALUE
    assert call(workspace=None) == HIP_ERROR_INVALID_VALUE


def test_batch_engine_and_trace_entry_points_check_their_arguments(lib):
    """mk_set_batch_engine takes 0, 1 or 2 only; mk_set_batch_trace refuses a buffer smaller than
    mk_batch_trace_bytes() (one stamp row per workgroup and layer) and accepts NULL (trace off).
    Neither launches anything."""
    assert lib.mk_set_batch_engine(3) == HIP_ERROR_INVALID_VALUE
    assert lib.mk_set_batch_engine(-1) == HIP_ERROR_INVALID_VALUE
    for e in (1, 2, 0):
        assert lib.mk_set_batch_engine(e) == HIP_SUCCESS
    lib.mk_batch_trace_bytes.restype = ctypes.c_size_t
    lib.mk_set_batch_trace.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    need = lib.mk_batch_trace_bytes()
    assert need == 256 * 33 * 24 * 8
    assert lib.mk_set_batch_trace(ctypes.c_void_p(16), need - 8) == HIP_ERROR_INVALID_VALUE
    assert lib.mk_set_batch_trace(None, 0) == HIP_SUCCESS

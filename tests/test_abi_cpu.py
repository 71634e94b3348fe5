"""C ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments with a status and a message before
any device work."""

import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (binds the library's HIP runtime dependency to torch's)

from megaslide_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "megaslide_dsa3d.h")

pytestmark = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH),
                                reason="HIP library not built (python -m megaslide_amd.csrc.build)")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(msd_[a-z0-9_]+)\s*\(", text)))


def test_exports_match_header():
    lib = _lib.load()
    declared = header_functions()
    assert declared == sorted(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version():
    assert _lib.load().msd_abi_version() == _lib.ABI_VERSION == 5


def _desc(**kw):
    d = dict(B=1, T=4, H=5, W=6, num_heads=2, head_dim=64, kt=3, kh=7, kw=7, dtype=0,
             q_stride=128, k_stride=128, v_stride=128, offset_scale=1.0, softmax_scale=0.125)
    d.update(kw)
    return _lib.DsaDesc(**d)


def _fwd(desc, ptrs=(16, 16, 16, 16, 16), lse=None, extra=(None, None)):
    lib = _lib.load()
    return lib.msd_dsa3d_fwd(ctypes.byref(desc) if desc is not None else None, *ptrs[:4], *extra,
                             ptrs[4], lse, None)


def test_null_desc_rejected():
    lib = _lib.load()
    assert lib.msd_dsa3d_fwd(None, 16, 16, 16, 16, None, None, 16, None, None) == -1
    assert b"desc is NULL" in lib.msd_last_error()


@pytest.mark.parametrize("field,value,code,needle", [
    ("T", 0, -1, b"bad shape"),
    ("num_heads", 0, -1, b"bad heads"),
    ("head_dim", 4096, -2, b"head_dim"),
    ("kt", 0, -1, b"bad window"),
    ("dtype", 7, -2, b"dtype"),
    ("q_stride", 64, -1, b"strides"),
    ("dropout_p", 1.0, -1, b"dropout_p"),
    ("dropout_p", -0.1, -1, b"dropout_p"),
    ("dropout_p", float("nan"), -1, b"dropout_p"),
    ("extra_g", -1, -1, b"extra_g"),
    ("extra_g", 5000, -1, b"extra_g"),
    ("dkv_accum", 2, -1, b"dkv_accum"),
    ("dkv_accum", 1, -1, b"bf16 storage"),   # scaled fp16 sums: bf16 only (dtype 0 here)
])
def test_bad_desc_fields(field, value, code, needle):
    rc = _fwd(_desc(**{field: value}))
    assert rc == code
    assert needle in _lib.load().msd_last_error()


def test_null_and_misaligned_pointers():
    lib = _lib.load()
    assert _fwd(_desc(), ptrs=(16, None, 16, 16, 16)) == -1
    assert b"NULL" in lib.msd_last_error()
    assert _fwd(_desc(), ptrs=(16, 18, 16, 16, 16)) == -3  # fp32 needs 4-byte alignment
    assert _fwd(_desc(dtype=1), ptrs=(16, 17, 16, 16, 16)) == -3


def test_extra_keys_need_their_pointers():
    lib = _lib.load()
    assert _fwd(_desc(extra_g=4)) == -1 and b"extra_k" in lib.msd_last_error()
    assert _fwd(_desc(extra_g=4), extra=(16, 24)) == -3  # 16-byte aligned rows


def test_empty_batch_is_a_no_op():
    assert _fwd(_desc(B=0)) == 0


def test_workspace_size_and_check():
    lib = _lib.load()
    rows = 2 * 4 * 5 * 6
    # head_dim 16: direct kernels only, dK/dV fp32 accumulators
    d16 = _desc(B=2, head_dim=16, q_stride=32, k_stride=32, v_stride=32)
    assert lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(d16)) == 2 * rows * 32 * 4
    # head_dim 64: the tiled backward keeps p and ds of every tap: two fp32
    # arrays for fp32 storage, which adds dK/dV up in its outputs (the direct
    # kernels' accumulators are less than p and ds, and the larger of the two
    # is asked for); for bf16 one word of two fp16 per tap plus one fp32 per
    # (token, head), beside fp32 rows (which also hold the fp16 accumulators),
    # then the scale bounds (8 floats from each of 256 blocks) and 32 bytes of
    # scales and overflow flag
    taps = rows * 2 * 147 * 4
    records = 256 * 8 * 4
    # bf16 with fp32 dK/dV accumulation also holds the column-streaming
    # kernel's tap records (16 bytes per tap), 32-int headers and transposed
    # q/dO (bf16) of every (head, one-frame tile), a list of one int per
    # (head, 4x4 column) after its count, and 8 work counters; T=4, H=5, W=6:
    # 4 frames x 2 x 2 tiles
    tiles, cols = 2 * 4 * 2 * 2 * 2, 2 * 2 * 2 * 2
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    stream = up(2 * rows * 128 * 4 + taps + rows * 2 * 4 + records + 32)
    stream = up(stream + tiles * 147 * 16 * 16)
    stream = up(stream + tiles * 32 * 4)
    stream = up(stream + tiles * 2 * 64 * 16 * 2) + (cols + 1 + 8) * 4
    for dtype, accum, want in ((0, 0, max(2 * rows * 128 * 4, 2 * taps)),
                               (1, 1, 2 * rows * 128 * 4 + taps + rows * 2 * 4 + records + 32),
                               (1, 0, stream)):
        d = _desc(B=2, dtype=dtype, dkv_accum=accum)
        need = lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(d))
        assert need == want
    # with extra keys the tiled backward also keeps their fp32 part of dq and
    # the fp32 Delta per (token, head)
    dx = _desc(B=2, dtype=1, extra_g=8)
    G, D = 8, 128
    want = (2 * rows * D * 4 + 2 * 2 * G * D * 4 + taps + rows * 2 * 4)
    want = (want + 255) // 256 * 256 + 2 * rows * 2 * G * 2
    want = (want + 255) // 256 * 256 + rows * D * 4
    want = (want + 255) // 256 * 256 + rows * 2 * 4
    want = (want + 255) // 256 * 256 + records + 32
    assert lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(dx)) == want
    rc = lib.msd_dsa3d_bwd(ctypes.byref(d), *([16] * 4), None, None, *([16] * 3), None,
                           *([16] * 4), None, None, 16, need - 1, None)
    assert rc == -4 and b"workspace" in lib.msd_last_error()
    assert lib.msd_dsa3d_bwd_workspace_size(None) == 0


def test_dwconv_validation():
    lib = _lib.load()
    d = _lib.ConvDesc(1, 4, 5, 6, 32, 3, 7, 7, 0, 0)
    bad = _lib.ConvDesc(1, 4, 5, 6, 32, 3, 6, 7, 0, 0)  # even kernel
    assert lib.msd_dwconv3d_fwd(ctypes.byref(bad), 16, 16, None, 16, None, None) == -2
    assert b"odd" in lib.msd_last_error()
    assert lib.msd_dwconv3d_fwd(ctypes.byref(d), 16, None, None, 16, None, None) == -1
    # the saved pre-activation belongs to the GELU form only
    assert lib.msd_dwconv3d_fwd(ctypes.byref(d), 16, 16, None, 16, 16, None) == -1
    assert b"act = 1" in lib.msd_last_error()
    gelu = _lib.ConvDesc(2, 4, 5, 6, 32, 3, 3, 3, 1, 1)
    assert lib.msd_dwconv3d_fwd(ctypes.byref(gelu), 16, 16, None, 16, 17, None) == -3
    ws = lib.msd_dwconv3d_bwd_workspace_size(ctypes.byref(gelu))
    assert ws >= 4 * (2 * 4 * 5 * 6 * 32 + 32 * 28)
    assert lib.msd_dwconv3d_bwd(ctypes.byref(gelu), 16, 16, 16, None, 16, 16, 16, 16, None, ws,
                                None) == -4


def test_module_rejects_cpu_tensors():
    from megaslide_amd import DeformableSlideAttention3D
    m = DeformableSlideAttention3D(16, 2, kernel_size=(3, 3, 3))
    with pytest.raises(RuntimeError, match="ROCm"):
        m(torch.randn(1, 8, 16), (2, 2, 2))
    with pytest.raises(AssertionError):
        m(torch.randn(1, 9, 16), (2, 2, 2))


def test_noalloc_scratch_limit_and_rejection():
    """The no-allocation backward's scratch maximum is the header's constant,
    and a call needing more is rejected by the size check, before any device
    call (the pointers here are never dereferenced)."""
    text = open(HEADER).read()
    m = re.search(r"#define MSD_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES
    lib = _lib.load()
    big = _desc(B=1, T=64, H=32, W=32, num_heads=16, dtype=1, q_stride=1024, k_stride=1024,
                v_stride=1024)
    assert lib.msd_dsa3d_bwd_workspace_size(ctypes.byref(big)) > _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.msd_dsa3d_bwd_noalloc(ctypes.byref(big), *([16] * 4), None, None, *([16] * 3), None,
                                   *([16] * 4), None, None, None)
    assert rc == -4 and b"maximum" in lib.msd_last_error()

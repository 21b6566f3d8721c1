"""The C-ABI library on a CPU-only host: it loads, exports every function that
include/fal_api.h declares, and rejects bad arguments with the documented status
codes and messages before touching a GPU (the reference raises the same
conditions through TORCH_CHECK, csrc/flash_attn_legacy.cpp:48-60,115-120,201-217).
"""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fal_api.h")

FAL_OK, FAL_ERR_INVALID, FAL_ERR_UNSUPPORTED, FAL_ERR_LAUNCH, FAL_ERR_WORKSPACE = range(5)


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fal_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def ext():
    from flash_attn_legacy import hip_ext
    return hip_ext


@pytest.fixture(scope="module")
def lib(ext):
    return ext._lib


def test_header_declares_the_expected_entry_points():
    names = header_functions()
    for n in ("fal_fwd", "fal_fwd_varlen", "fal_bwd", "fal_bwd_varlen", "fal_decode",
              "fal_last_error", "fal_version", "fal_device_supported"):
        assert n in names
    for n in ("fal_fwd", "fal_fwd_varlen", "fal_bwd", "fal_bwd_varlen", "fal_decode"):
        assert n + "_bf16" in names


def test_library_exports_every_header_symbol(ext):
    dll = ctypes.CDLL(ext.library_path())
    for name in header_functions():
        assert hasattr(dll, name), f"{name} declared in fal_api.h but not exported"
    assert set(ext.SYMBOLS) == set(header_functions())


def test_version(ext):
    assert ext.version().startswith("0.5.0")


def s3(*v):
    return (ctypes.c_int64 * 3)(*v)


def fwd(lib, d=64, hq=4, hkv=2, ptr=4096, strides=None, lse=4096, bf16=False):
    st = strides or s3(4 * 16 * d, 16 * d, d)
    return (lib.fal_fwd_bf16 if bf16 else lib.fal_fwd)(ctypes.c_void_p(ptr), ctypes.c_void_p(ptr), ctypes.c_void_p(ptr), ctypes.c_void_p(ptr),
                       ctypes.c_void_p(lse) if lse else None, 1, hq, hkv, 16, 16, d, st, st, st, st, 0.125, 1,
                       None, 0, None)


def test_forward_rejects_head_dim(lib):
    assert fwd(lib, d=48) == FAL_ERR_UNSUPPORTED
    assert b"head_dim must be 32, 64, 96, 128, or 256, got 48" in lib.fal_last_error()


def test_bf16_forward_checks_like_fp16(lib):
    """The bf16 entry point validates its arguments exactly as the fp16 one does."""
    for kw, code, msg in ((dict(d=48), FAL_ERR_UNSUPPORTED, b"head_dim must be"),
                          (dict(hq=6, hkv=4), FAL_ERR_INVALID, b"divisible"),
                          (dict(ptr=0), FAL_ERR_INVALID, b"null"),
                          (dict(lse=0), FAL_ERR_INVALID, b"lse")):
        assert fwd(lib, bf16=True, **kw) == code
        assert msg in lib.fal_last_error()
        assert fwd(lib, bf16=False, **kw) == code


def test_forward_rejects_gqa_ratio(lib):
    assert fwd(lib, hq=6, hkv=4) == FAL_ERR_INVALID
    assert b"divisible" in lib.fal_last_error()


def test_forward_rejects_null_misaligned_and_strides(lib):
    assert fwd(lib, ptr=0) == FAL_ERR_INVALID
    assert b"null pointer" in lib.fal_last_error()
    assert fwd(lib, ptr=4098) == FAL_ERR_INVALID
    assert b"16-byte aligned" in lib.fal_last_error()
    assert fwd(lib, strides=s3(1000, 100, 66)) == FAL_ERR_INVALID
    assert b"multiple of 8" in lib.fal_last_error()
    assert fwd(lib, lse=0) == FAL_ERR_INVALID


def test_forward_split_workspace(lib):
    """Grids far smaller than the GPU with long key ranges (one head of 16384 rows) split
    the key range and need a workspace for the partial outputs; C1 (2 x 8 heads x 1024
    rows, where the partials would cost more than the shorter chain saves) and C2 need
    none, and neither do short key ranges."""
    one = lib.fal_fwd_workspace_size(1, 1, 16384, 16384, 64, 1)
    assert one >= 2 * 16384 * 66 * 4                  # at least two splits of every row
    assert lib.fal_fwd_workspace_size(2, 8, 1024, 1024, 64, 1) == 0
    assert lib.fal_fwd_workspace_size(4, 32, 4096, 4096, 128, 1) == 0
    assert lib.fal_fwd_workspace_size(2, 8, 128, 128, 64, 1) == 0
    st = s3(16384 * 64, 16384 * 64, 64)
    p = ctypes.c_void_p(4096)
    rc = lib.fal_fwd(p, p, p, p, p, 1, 1, 1, 16384, 16384, 64, st, st, st, st, 0.125, 1, None, 0, None)
    assert rc == FAL_ERR_WORKSPACE
    assert b"workspace needs" in lib.fal_last_error()


def test_workspace_sizes_and_checks(lib):
    # d 32/64/96: delta only (the query-outer dQ kernel needs no fp32 accumulator);
    # d 128: delta + the tile-major (-L*log2e/c, -D) array of the pipelined dK/dV kernel,
    # 64-row tiles (rounded up); d 256: delta + the fp32 dQ accumulator of the atomic kernel
    rows = 2 * 16 * 2048
    for d in (32, 64, 96):
        assert rows * 4 <= lib.fal_bwd_workspace_size(2, 16, 2048, d) < rows * 4 + 4096
    assert rows * 12 <= lib.fal_bwd_workspace_size(2, 16, 2048, 128) < rows * 12 + 4096
    assert lib.fal_bwd_workspace_size(1, 1, 65, 128) >= 65 * 4 + 2 * 128 * 4
    assert lib.fal_bwd_workspace_size(2, 16, 2048, 256) >= rows * 257 * 4
    # small problems (<= 64 sequences, <= 16384 query tokens) derive their work items in
    # the kernel: no workspace; larger ones get a (sequence, tile) list
    assert lib.fal_fwd_varlen_workspace_size(16, 1504, 1024, 64) == 0
    assert lib.fal_fwd_varlen_workspace_size(64, 16384, 4096, 128) == 0
    assert lib.fal_fwd_varlen_workspace_size(65, 6400, 256, 128) >= (6400 // 256 + 65) * 8
    assert lib.fal_fwd_varlen_workspace_size(16, 35901, 4096, 128) >= (35901 // 256 + 16) * 8
    assert lib.fal_decode_workspace_size(32, 32, 8, 32768, 128) > 0
    st = s3(0, 64, 256)
    cu = ctypes.c_void_p(4096)
    p = ctypes.c_void_p(4096)
    rc = lib.fal_fwd_varlen(p, p, p, p, p, cu, cu, 100, 6400, 6400, 4, 4, 64, 64, 64, st, st, st, st, 0.1, 1,
                            p, 8, None)
    assert rc == FAL_ERR_WORKSPACE
    assert b"workspace needs" in lib.fal_last_error()


def test_decode_rejects_large_groups(lib):
    p = ctypes.c_void_p(4096)
    st = s3(64 * 128, 128, 0)
    rc = lib.fal_decode(p, p, p, p, None, 0, p, None, 1, 64, 1, 128, 16, st, st, st, st, 0.1, p, 1 << 20, None)
    assert rc == FAL_ERR_UNSUPPORTED
    assert b"at most 32" in lib.fal_last_error()


def test_error_message_cleared_on_success(lib, ext):
    fwd(lib, d=48)
    assert lib.fal_last_error() != b""
    # batch == 0 is a valid no-op (no GPU work is enqueued)
    st = s3(0, 0, 64)
    p = ctypes.c_void_p(4096)
    assert lib.fal_fwd(p, p, p, p, p, 0, 4, 2, 16, 16, 64, st, st, st, st, 0.125, 0, None, 0, None) == FAL_OK
    assert lib.fal_last_error() == b""


def test_device_supported_without_gpu(ext):
    import torch
    if torch.cuda.is_available():
        pytest.skip("GPU host")
    assert ext.device_supported(0) is False


def test_missing_library_fails_loudly(tmp_path):
    """No CPU fallback: without the HIP library the package does not import."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "try:\n    import flash_attn_legacy\nexcept ImportError as e:\n"
            "    print('IMPORTERROR', e)\nelse:\n    print('IMPORTED')\n") % os.path.join(ROOT, "flash-attention-legacy_amd")
    env = dict(os.environ, FLASH_ATTN_LEGACY_LIB=str(tmp_path / "missing.so"))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert "IMPORTERROR" in r.stdout and "HIP library not found" in r.stdout, r.stdout + r.stderr

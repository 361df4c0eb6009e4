"""The C ABI: include/mhc_hip.h <-> libmhc_hip.so <-> the ctypes table (CPU only).

Loading the library and calling its pure-host entry points (version, error
text, argument validation) needs no GPU; nothing here launches a kernel.
"""

import ctypes
import re
from pathlib import Path

import pytest

from mhc_mlx_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mhc_hip.h"


def _declarations():
    """{name: parameter count} of every function declared in the header."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(mhc_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libmhc_hip.so not built")
    return _lib.load()


def test_header_declares_the_ctypes_table():
    decl = _declarations()
    assert set(decl) == set(_lib.SIGNATURES), set(decl) ^ set(_lib.SIGNATURES)
    for name, (args, _res) in _lib.SIGNATURES.items():
        assert len(args) == decl[name], name


def test_library_exports_every_declared_symbol(lib):
    for name in _declarations():
        assert hasattr(lib, name), name


def test_abi_version_and_error_text(lib):
    assert lib.mhc_abi_version() == 1
    assert isinstance(lib.mhc_last_error(), bytes)


@pytest.mark.parametrize("n,C,T", [(0, 16, 1), (65, 16, 1), (4, 0, 1), (4, 16, -1)])
def test_fused_fwd_rejects_bad_shapes_on_the_host(lib, n, C, T):
    rc = lib.mhc_fused_fwd(None, 1, None, 0, None, None, 0, _lib.H_RAW, None, None, 1, None, T, n, C,
                           ctypes.c_float(1e-6), None)
    assert rc == -1
    assert lib.mhc_last_error()


def test_fused_fwd_rejects_mixed_parameter_modes(lib):
    rc = lib.mhc_fused_fwd(None, 1, None, 16, None, None, 0, _lib.H_RAW, None, None, 1, None, 8, 4, 16,
                           ctypes.c_float(1e-6), None)
    assert rc == -1
    assert b"per-token" in lib.mhc_last_error()


def test_fused_fwd_rejects_bad_output_dtype(lib):
    dummy = ctypes.c_void_p(16)
    rc = lib.mhc_fused_fwd(dummy, 1, dummy, 0, dummy, dummy, 0, _lib.H_RAW, dummy, dummy, 2, None, 8, 4, 16,
                           ctypes.c_float(1e-6), None)
    assert rc == -1
    assert b"out_dtype" in lib.mhc_last_error()


def test_zero_tokens_is_a_no_op(lib):
    rc = lib.mhc_fused_fwd(None, 1, None, 0, None, None, 0, _lib.H_RAW, None, None, 1, None, 0, 4, 16,
                           ctypes.c_float(1e-6), None)
    assert rc == 0


def test_sinkhorn_rejects_bad_arguments(lib):
    assert lib.mhc_sinkhorn_fwd(None, None, 1, 0, 20, ctypes.c_float(1e-5), None) == -1
    assert lib.mhc_sinkhorn_fwd(None, None, 1, 4, -1, ctypes.c_float(1e-5), None) == -1
    assert lib.mhc_sinkhorn_fwd(None, None, 0, 4, 20, ctypes.c_float(1e-5), None) == 0
    assert lib.mhc_sinkhorn_fwd(None, None, 2, 4, 20, ctypes.c_float(1e-5), None) == -1


def test_layer_bwd_rejects_null_gradients(lib):
    dummy = ctypes.c_void_p(16)
    rc = lib.mhc_layer_bwd(dummy, 1, dummy, 1, dummy, dummy, dummy, dummy, dummy, dummy, None, None, None, None,
                           None, 0, 8, 4, 16, 0, 20, ctypes.c_float(1e-6), None)
    assert rc == -1
    assert b"gradient" in lib.mhc_last_error()


def test_check_maps_status_to_exceptions(lib):
    _lib.check(0, "ok")
    lib.mhc_sinkhorn_fwd(None, None, 1, 0, 20, ctypes.c_float(1e-5), None)
    with pytest.raises(ValueError):
        _lib.check(-1, "mhc_sinkhorn_fwd")
    with pytest.raises(_lib.MHCError):
        _lib.check(1, "x")


def test_residual_add_agg_rejects_bad_arguments_on_the_host(lib):
    assert lib.mhc_residual_add_agg_fwd(None, None, 1, None, _lib.H_ACTIVATED, None, 0, None, 4, 0, 8, None) == -1
    assert lib.mhc_residual_add_agg_fwd(None, None, 1, None, 7, None, 0, None, 4, 4, 8, None) == -1
    assert lib.mhc_residual_add_agg_fwd(None, None, 1, None, _lib.H_ACTIVATED, None, 0, None, 4, 4, 8, None) == -1
    assert b"null pointer" in lib.mhc_last_error()
    assert lib.mhc_residual_add_agg_bwd(None, None, 9, None, 0, None, None, _lib.H_ACTIVATED, None, None, None,
                                        None, 0, 4, 4, 8, None) == -1


def test_sinkhorn_state_is_for_n16_to_64_and_checked_on_the_host(lib, knobs):
    # n = 16: the block layout's compact record whatever layout the unrecorded calls use: per matrix
    # 32 floats per iteration (row and column sums) and 32 per 5-iteration VJP segment after the first
    # (the scales at its start), at least 32
    def rec16(B, iters):
        nseg = -(-iters // 5)
        return B * 32 * 4 * max(1, iters + max(nseg - 1, 0)) + 256

    assert lib.mhc_sinkhorn_state_bytes(8, 16, 20) == rec16(8, 20) == 8 * 23 * 128 + 256
    assert lib.mhc_sinkhorn_state_bytes(3, 16, 7) == rec16(3, 7) == 3 * 8 * 128 + 256
    assert lib.mhc_sinkhorn_state_bytes(2, 16, 5) == rec16(2, 5) == 2 * 5 * 128 + 256
    assert lib.mhc_sinkhorn_state_bytes(2, 16, 0) == rec16(2, 0) == 2 * 128 + 256
    knobs("MHC_SK16_CPL", 4)
    assert lib.mhc_sinkhorn_state_bytes(8, 16, 20) == rec16(8, 20)
    knobs("MHC_SK16_CPL", None)
    # block layout (16 < n <= 64): six vectors of next_pow2(n) floats per matrix and iteration
    assert lib.mhc_sinkhorn_state_bytes(8, 32, 20) == 8 * 20 * 6 * 32 * 4 + 256
    assert lib.mhc_sinkhorn_state_bytes(3, 24, 7) == 3 * 7 * 6 * 32 * 4 + 256
    assert lib.mhc_sinkhorn_state_bytes(1, 64, 0) == 1 * 1 * 6 * 64 * 4 + 256
    assert lib.mhc_sinkhorn_state_bytes(8, 4, 20) == 0
    assert lib.mhc_sinkhorn_state_bytes(8, 65, 20) == 0
    assert lib.mhc_sinkhorn_state_bytes(0, 16, 20) == 0
    knobs("MHC_SK16", 0)
    assert lib.mhc_sinkhorn_state_bytes(8, 16, 20) == 0
    knobs("MHC_SK16", None)
    knobs("MHC_SK16_RECORD", 0)
    assert lib.mhc_sinkhorn_state_bytes(8, 16, 20) == 0
    assert lib.mhc_sinkhorn_state_bytes(8, 32, 20) > 0
    knobs("MHC_SK16_RECORD", None)
    knobs("MHC_SK_BLK_RECORD", 0)
    assert lib.mhc_sinkhorn_state_bytes(8, 32, 20) == 0
    assert lib.mhc_sinkhorn_state_bytes(8, 16, 20) > 0
    knobs("MHC_SK_BLK_RECORD", None)
    fake = ctypes.c_void_p(4096)  # never dereferenced: every call below is rejected on the host
    eps = ctypes.c_float(1e-6)
    assert lib.mhc_sinkhorn_fwd_record(fake, fake, fake, 1 << 20, 8, 4, 20, eps, None) == -1
    assert b"16 <= n <= 64" in lib.mhc_last_error()
    assert lib.mhc_sinkhorn_bwd_recorded(fake, fake, fake, fake, 1 << 20, 8, 65, 20, eps, None) == -1
    assert lib.mhc_sinkhorn_fwd_record(fake, fake, fake, 100, 8, 16, 20, eps, None) == -1
    assert b"smaller" in lib.mhc_last_error()
    assert lib.mhc_sinkhorn_fwd_record(fake, fake, fake, 8 * 20 * 768 - 1, 8, 32, 20, eps, None) == -1
    assert b"smaller" in lib.mhc_last_error()
    assert lib.mhc_sinkhorn_bwd_recorded(fake, fake, fake, None, 1 << 20, 8, 16, 20, eps, None) == -1
    assert lib.mhc_sinkhorn_bwd_recorded(fake, fake, fake, fake, 1 << 20, 8, 16, -1, eps, None) == -1
    assert lib.mhc_sinkhorn_fwd_record(fake, fake, fake, 0, 0, 16, 20, eps, None) == 0  # empty batch


def test_torch_binding_loads_and_exports_the_layer_calls():
    """_mhc_torch.so (csrc/torch_ext.cpp) loads after libmhc_hip.so and exports MHCLayer's two calls."""
    from mhc_mlx_amd import _ext

    mod = _ext.load()
    assert callable(mod.layer_apply) and callable(mod.layer_forward_nograd) and callable(mod.module_forward) and callable(mod.module_call)
    assert _ext.load() is mod

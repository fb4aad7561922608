"""The C-ABI library: loads, exports every declared symbol, and rejects bad
arguments before touching a device (no compute calls here)."""
import ctypes
import os
import re

import pytest

from amd_optimization_challenge_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    with open(os.path.join(ROOT, "include", "mla_mi355x.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int64_t|int)\s+(mla_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    syms = declared_symbols()
    assert len(syms) >= 10
    assert sorted(_lib.SIGNATURES) == syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.mla_abi_version() == 2


def test_argument_errors_without_device():
    lib = _lib.load()
    n = ctypes.c_int64(0)
    assert lib.mla_workspace_bytes(4, 24, 0, ctypes.byref(n)) == _lib.MLA_ERR_UNSUPPORTED
    assert b"num_heads" in lib.mla_last_error()
    assert lib.mla_workspace_bytes(0, 16, 0, ctypes.byref(n)) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_workspace_bytes(4, 128, 1, ctypes.byref(n)) == _lib.MLA_ERR_UNSUPPORTED
    assert lib.mla_workspace_bytes(4, 16, 7, ctypes.byref(n)) == _lib.MLA_ERR_INVALID_ARGUMENT
    # the bf16 cache (a16w16): 16 heads, bf16 Q through mla_decode_fwd only
    assert lib.mla_workspace_bytes(4, 128, 3, ctypes.byref(n)) == _lib.MLA_ERR_UNSUPPORTED
    assert lib.mla_decode(None, None, None, 1152, None, 0, None, 0, None, None, None, 4, 16, 0.1, 3, None, 0,
                          None, None, None) == _lib.MLA_ERR_UNSUPPORTED
    assert lib.mla_pack_mxfp4(None, 4, 33, 66, None, 16, None, 2, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_quant_fp8_per_tensor(None, 0, None, None, None, 0, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_selftest(0, None, None, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    # neighbouring steps: bad sizes, null pointers, fp8 output without its workspace
    assert lib.mla_absorb_q(16, 16, 16, 0, 16, 16, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_absorb_q(None, 16, 16, 4, 16, 16, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_v_up_proj(16, 16, 4, 257, 16, None, None, None, 0, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert b"256" in lib.mla_last_error()
    assert lib.mla_v_up_proj(16, 16, 4, 16, 16, 16, 16, None, 0, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_v_up_proj(16, 16, 4, 16, 16, 16, 16, 16, 4096, None) == _lib.MLA_ERR_WORKSPACE_TOO_SMALL
    # append: no cache, negative n, fp8 cache without its scale, short scale stride
    assert lib.mla_append_kv(None, 4, 1152, None, None, 0, None, None, 0, None, 0, None,
                             None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_append_kv(None, -1, 1152, None, 16, 576, 16, None, 0, None, 0, None,
                             None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_append_kv(16, 4, 1152, None, 16, 576, None, None, 0, None, 0, None,
                             None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_append_kv(16, 4, 1152, None, None, 0, None, 16, 288, 16, 17, None,
                             None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert b"18" in lib.mla_last_error()
    assert lib.mla_append_kv(16, 29826162, 1152, None, 16, 576, 16, None, 0, None, 0, None,
                             None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_append_kv(None, 0, 0, None, 16, 0, None, None, 0, None, 0, None, None) == _lib.MLA_OK
    with pytest.raises(_lib.MlaLibraryError):
        _lib.check(lib.mla_workspace_bytes(4, 24, 0, ctypes.byref(n)), "mla_workspace_bytes")
    # q_seq_len must divide the query rows (checked before any device call)
    assert lib.mla_plan(None, 6, 4, 16, 0, None, 0, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_decode_fwd(None, None, 576, None, 0, None, 0, None, None, None, 6, 4, 16, 0.1, 0, None, 0,
                              None, None, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    # page-table expansion: bad batch / page size, 2^31-row overflow, null pointers
    assert lib.mla_expand_pages(None, None, None, 0, 16, 0, None, None, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_expand_pages(None, None, None, 4, 0, 0, None, None, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert lib.mla_expand_pages(16, 16, 16, 4, 64, 1 << 25, 16, 16, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    assert b"2^31" in lib.mla_last_error()
    assert lib.mla_expand_pages(None, None, None, 4, 8, 10, None, None, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    # the a16w8 route: 16 heads and the fp8 cache only
    assert lib.mla_decode_fwd_a16w8(None, None, 576, None, 0, None, 0, None, None, None, 4, 1, 128, 0.1, 0,
                                    None, 0, None, None, None) == _lib.MLA_ERR_UNSUPPORTED
    assert lib.mla_decode_fwd_a16w8(None, None, 288, None, 18, None, 0, None, None, None, 4, 1, 16, 0.1, 1,
                                    None, 0, None, None, None) == _lib.MLA_ERR_UNSUPPORTED
    assert lib.mla_decode_fwd_a16w8(None, None, 576, None, 0, None, 0, None, None, None, 4, 1, 16, 0.1, 0,
                                    None, 0, None, None, None) == _lib.MLA_ERR_INVALID_ARGUMENT
    # the no-alloc variant: stated scratch size, shape errors before any device call
    assert lib.mla_noalloc_scratch_bytes() == 64 << 20
    assert lib.mla_decode_fwd_noalloc(None, None, 576, None, 0, None, 0, None, None, None, 4, 1, 24, 0.1, 0,
                                      None, None, None) == _lib.MLA_ERR_UNSUPPORTED


def test_custom_kernel_rejects_unsupported_configs_before_launch():
    import torch

    from amd_optimization_challenge_amd import custom_kernel

    q = torch.zeros((2, 16, 576), dtype=torch.bfloat16)
    indptr = torch.tensor([0, 1, 2], dtype=torch.int32)
    with pytest.raises(ValueError):  # 2 query rows cannot be 2 sequences x q_seq_len 2
        custom_kernel((q, {}, indptr, indptr, {"q_seq_len": 2}))
    with pytest.raises(ValueError):
        custom_kernel((q, {}, indptr, indptr, {"num_heads": 128}))
    with pytest.raises(ValueError):  # CPU tensors: the HIP path refuses them
        custom_kernel((q, {"fp8": (q, q)}, indptr, indptr, {}))

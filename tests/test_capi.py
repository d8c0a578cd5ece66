"""The C-ABI library: loads, exports every declared symbol, rejects bad
arguments with a message (host-side checks only; no GPU needed)."""
import ctypes
import os
import re

import pytest

import qwq4

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qw", "q4ops.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(qw_\w+)\s*\(", src))


def test_exports_every_declared_symbol():
    L = qwq4.lib()
    names = declared()
    assert names == set(qwq4.SYMBOLS)
    for n in names:
        assert getattr(L, n) is not None


def test_abi_version():
    assert qwq4.lib().qw_q4_abi_version() == 5


@pytest.mark.parametrize("call", [
    lambda L: L.qw_q4_gemv(None, None, None, None, 0, 4096, None, 4096, 0, 4096, 4096, 1, 0, 0, None),
    lambda L: L.qw_q4_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 0, 4096,
                           ctypes.c_void_p(256), 4096, 0, 4096, 4000, 1, 0, 0, None),
    lambda L: L.qw_q4_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 0, 4096,
                           ctypes.c_void_p(256), 4096, 0, 4096, 4096, 33, 0, 0, None),
    lambda L: L.qw_moe_route(ctypes.c_void_p(256), 4, 256, 0, 0, *([ctypes.c_void_p(256)] * 11), None),
    lambda L: L.qw_moe_combine(None, 0, None, None, None, 0, 1, 8, 4096, None, 1, None),
    lambda L: L.qw_q4_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 0, 4096,
                           ctypes.c_void_p(256), 4096, 0, 4008, 4096, 1, 0, 0, None),  # N % 16
    lambda L: L.qw_q4_gemm(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 0, 4096, 4096,
                           ctypes.c_void_p(256), 4096, 1, 4096, 4096, None, 0, None),
    lambda L: L.qw_q4_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(264), 0, 4096,
                           ctypes.c_void_p(256), 4096, 0, 4096, 4096, 1, 0, 0, None),  # x not 16-byte aligned
    lambda L: L.qw_moe_experts_gemv(*([ctypes.c_void_p(256)] * 9), 256, 4096, 1536, *([ctypes.c_void_p(256)] * 5),
                                    0, 33, 8, ctypes.c_void_p(256), ctypes.c_void_p(256), 0, None),  # T > 32
    lambda L: L.qw_moe_experts_grouped(*([ctypes.c_void_p(256)] * 9), 256, 4096, 1536,
                                       *([ctypes.c_void_p(256)] * 6), 0, 4096, 8, ctypes.c_void_p(256),
                                       ctypes.c_void_p(256), 0, ctypes.c_void_p(256), 0, None),  # workspace too small
    lambda L: L.qw_moe_decode(ctypes.c_void_p(256), 0, ctypes.c_void_p(256), 0, 33, 256, 8,
                              *([ctypes.c_void_p(256)] * 9), 4096, 1536, None, ctypes.c_void_p(256), 1,
                              *([ctypes.c_void_p(256)] * 6), 0, ctypes.c_void_p(256), 1 << 30, None),  # T > 32
    lambda L: L.qw_i8_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), 32, ctypes.c_void_p(256), 96,
                           ctypes.c_void_p(256), 64, 0, 64, 96, 1, 0, 0, None),  # K % 64
    lambda L: L.qw_i8_tile(ctypes.c_void_p(256), ctypes.c_void_p(256), 64, 4096, 64, ctypes.c_void_p(256),
                           ctypes.c_void_p(256), None),  # group 64
    lambda L: L.qw_i8_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), 64, ctypes.c_void_p(256), 128,
                           ctypes.c_void_p(256), 64, 0, 64, 128, 1, 0, 0, None),  # group 64
    lambda L: L.qw_i8_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), 32, ctypes.c_void_p(256), 128,
                           ctypes.c_void_p(256), 64, 0, 64, 128, 1, 8, 0, None),  # rpg < 16
    lambda L: L.qw_i8_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), 32, ctypes.c_void_p(256), 1024,
                           ctypes.c_void_p(256), 1296, 0, 1296, 1024, 2, 324, 0, None),  # xs < 4 slices
    lambda L: L.qw_w16_tile(ctypes.c_void_p(256), 96, 64, 48, ctypes.c_void_p(256), None),  # K % 32
    lambda L: L.qw_w16_tile(ctypes.c_void_p(256), 64, 64, 96, ctypes.c_void_p(256), None),  # ldw < K
    lambda L: L.qw_w16_gemv_tiled(ctypes.c_void_p(256), ctypes.c_void_p(256), 4096, 1, ctypes.c_void_p(256), 64, 0,
                                  64, 4096, 33, 0, 0, None),  # M > 32
    lambda L: L.qw_w16_gemv_tiled(ctypes.c_void_p(264), ctypes.c_void_p(256), 4096, 1, ctypes.c_void_p(256), 64, 0,
                                  64, 4096, 1, 0, 0, None),  # Wt not 16-byte aligned
    lambda L: L.qw_w16_swiglu_gemv_tiled(ctypes.c_void_p(256), ctypes.c_void_p(256), 97, 48, ctypes.c_void_p(256),
                                         64, 0, 64, 1, 0, None),  # n % 32
    lambda L: L.qw_w16_swiglu_gemv_tiled(ctypes.c_void_p(256), ctypes.c_void_p(256), 3073, 1536, ctypes.c_void_p(256),
                                         4096, 0, 4096, 33, 0, None),  # M > 32
    lambda L: L.qw_w16_swiglu_gemv_tiled(ctypes.c_void_p(256), ctypes.c_void_p(256), 3000, 1536, ctypes.c_void_p(256),
                                         4096, 0, 4096, 2, 0, None),  # ldv < 2n + 1
    lambda L: L.qw_q4_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 0, 4096,
                           ctypes.c_void_p(256), 1296, 0, 1296, 1024, 1, 8, 0, None),  # rpg < 16
    lambda L: L.qw_q4_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 0, 1024,
                           ctypes.c_void_p(256), 1296, 0, 1296, 1024, 2, 324, 0, None),  # xs < 4 slices
    lambda L: L.qw_q4_gemv(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 0, 4096,
                           ctypes.c_void_p(256), 4096, 0, 4096, 4096, 1, 16, 0, None),  # 256 slices > 64
    lambda L: L.qw_w16_gemv(ctypes.c_void_p(256), 1024, ctypes.c_void_p(256), 1024, 1, ctypes.c_void_p(256), 1296, 0,
                            1296, 1024, 2, 324, 0, None),  # xs < 4 slices
    lambda L: L.qw_q4_gemm(ctypes.c_void_p(256), ctypes.c_void_p(256), None, ctypes.c_void_p(256), 1, 4096, 4096,
                           ctypes.c_void_p(256), 4096, 3, 4096, 4096, None, 0, None),  # y_type 3
    lambda L: L.qw_moe_combine(ctypes.c_void_p(256), 1, ctypes.c_void_p(256), ctypes.c_void_p(256), None, 0, 1, 8,
                               4096, ctypes.c_void_p(256), 5, None),  # out_type 5
    lambda L: L.qw_moe_combine(ctypes.c_void_p(256), 1, ctypes.c_void_p(256), ctypes.c_void_p(256),
                               ctypes.c_void_p(260), 0, 1, 8, 4096, ctypes.c_void_p(256), 2, None),  # fp32 shared at 4 B
    lambda L: L.qw_moe_decode(ctypes.c_void_p(256), 0, ctypes.c_void_p(256), 0, 4, 256, 8,
                              *([ctypes.c_void_p(256)] * 9), 4096, 1536, None, ctypes.c_void_p(256), 7,
                              *([ctypes.c_void_p(256)] * 6), 1, ctypes.c_void_p(256), 1 << 30, None),  # out_type 7
    lambda L: L.qw_moe_decode(ctypes.c_void_p(256), 2, ctypes.c_void_p(256), 0, 4, 256, 8,
                              *([ctypes.c_void_p(256)] * 9), 4096, 1536, None, ctypes.c_void_p(256), 0,
                              *([ctypes.c_void_p(256)] * 6), 1, ctypes.c_void_p(256), 1 << 30, None),  # router_f16 2
    lambda L: L.qw_moe_decode_with_shared(ctypes.c_void_p(256), 1, ctypes.c_void_p(256), 1, 1, 256, 8, *([ctypes.c_void_p(256)] * 9), 4096, 1536,
                                          None, ctypes.c_void_p(256), 1536, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 2,
                                          *([ctypes.c_void_p(256)] * 6), 1, ctypes.c_void_p(256), 1 << 30, None),  # null sh_gu
    lambda L: L.qw_moe_decode_with_shared(ctypes.c_void_p(256), 1, ctypes.c_void_p(256), 1, 1, 256, 8, *([ctypes.c_void_p(256)] * 9), 4096, 1536,
                                          ctypes.c_void_p(256), ctypes.c_void_p(256), 1544, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 2,
                                          *([ctypes.c_void_p(256)] * 6), 1, ctypes.c_void_p(256), 1 << 30, None),  # Fs % 32
    lambda L: L.qw_moe_decode_with_shared(ctypes.c_void_p(256), 1, ctypes.c_void_p(256), 1, 1, 256, 8, *([ctypes.c_void_p(256)] * 9), 4096, 1536,
                                          ctypes.c_void_p(256), ctypes.c_void_p(256), 1536, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 2,
                                          *([ctypes.c_void_p(256)] * 6), 1, ctypes.c_void_p(256), 4096, None),  # workspace too small
])
def test_bad_arguments_are_rejected(call):
    L = qwq4.lib()
    assert call(L) == -1
    assert len(L.qw_q4_last_error()) > 0


def test_workspace_sizes():
    assert qwq4.lib().qw_w16_tiled_size(3073, 4096) == 3088 * 4096 * 2
    assert qwq4.gemm_workspace_size(4096, 4096) >= 4096 * 4096 * 2
    assert qwq4.lib().qw_q4_gemm_workspace_size(0, 4096) == 0

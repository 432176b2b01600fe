"""The C-ABI library loads without a GPU, exports every symbol include/strata_gfx950.h declares, and refuses bad
arguments before it touches the device (no compute call runs here)."""

import ctypes
import os
import re

import pytest

from strata_mlx_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "strata_gfx950.h")).read()
    return re.findall(r"^(?:int|int64_t)\s+(strata_\w+)\(", text, re.M)


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.library()
    names = declared()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.strata_abi_version() == 6


@pytest.mark.parametrize("kind, per, size", [("Q2_0", 64, 18), ("IQ3_S", 256, 110), ("IQ3_XXS", 256, 98),
                                             ("Q4_K", 256, 144), ("Q6_K", 256, 210), ("Q8_0", 32, 34),
                                             ("IQ4_NL", 32, 18), ("IQ4_XS", 256, 136), ("Q3_K", 256, 110),
                                             ("Q4_0", 32, 18), ("Q5_0", 32, 22)])
def test_block_info(kind, per, size):
    p, b = ctypes.c_int(), ctypes.c_int()
    assert _lib.library().strata_block_info(_lib.kind_id(kind), ctypes.byref(p), ctypes.byref(b)) == 0
    assert (p.value, b.value) == (per, size)


@pytest.mark.parametrize("kind", ["IQ2_S", "IQ2_XS", "IQ2_XXS", "IQ1_M"])
def test_types_without_kernels_are_refused(kind):
    lib = _lib.library()
    assert lib.strata_block_info(_lib.kind_id(kind), None, None) == _lib.ERR_KIND
    assert lib.strata_dequant(_lib.kind_id(kind), 1, 1, 1, 256, 1, 0, None) == _lib.ERR_KIND


def test_arguments_are_checked_before_any_launch():
    lib = _lib.library()
    q = _lib.kind_id("IQ3_S")
    assert lib.strata_dequant(q, 1, 1, 4, 100, 1, 0, None) == _lib.ERR_SHAPE  # 100 is not a block of 256
    assert lib.strata_dequant(q, 1, 1, 4, 256, 1, 2, None) == _lib.ERR_DTYPE  # bf16 out
    assert lib.strata_dequant(q, 0, 1, 4, 256, 0, 0, None) == _lib.ERR_ARG  # null pointers
    assert lib.strata_dequant(q, 0, 0, 4, 256, 0, 0, None) == _lib.OK  # nothing to do
    assert lib.strata_expert_matvec(q, 1, 4, 8, 256, 1, 6, 1, 1, 4, 1, None) == _lib.ERR_ARG  # 6 pairs, share 4
    assert lib.strata_expert_matvec(q, 1, 4, 8, 256, 1, 4, 1, 7, 1, 1, None) == _lib.ERR_DTYPE
    assert lib.strata_expert_matvec(q, 1, 4, 8, 16384, 1, 4, 1, 1, 1, 1, None) == _lib.ERR_SHAPE  # > 8192 cols
    assert lib.strata_expert_matvec(99, 1, 4, 8, 256, 1, 4, 1, 1, 1, 1, None) == _lib.ERR_KIND
    assert lib.strata_dense_matvec(q, 1, 8, 256, 1, 1, 1, 1, 2, None, 0, None) == _lib.ERR_DTYPE  # f16 -> bf16
    x3 = _lib.kind_id("IQ3_XXS")
    assert lib.strata_grouped_matmul(x3, 1, 4, 64, 256, 1, 2, None, 1, 1, 16, 1, None) == _lib.ERR_DTYPE  # bf16 a
    assert lib.strata_grouped_matmul(x3, 1, 4, 64, 256, 1, 0, 1, 1, 1, 16, 1, None) == _lib.ERR_ARG  # a_max on f32
    assert lib.strata_rows_to_f16(1, 4, 64, 7, 1, 1, None) == _lib.ERR_DTYPE
    assert lib.strata_rows_to_f16(0, 0, 64, 2, 0, 0, None) == _lib.OK  # no rows
    gu = lib.strata_prompt_gate_up_swiglu
    assert gu(_lib.kind_id("Q4_K"), 1, 1, 4, 64, 256, 1, None, 1, 1, 1, 16, 1, 1, None) == _lib.ERR_KIND
    assert gu(x3, 1, 1, 4, 64, 320, 1, None, 1, 1, 1, 16, 1, 1, None) == _lib.ERR_SHAPE  # not whole blocks
    assert gu(x3, 1, 1, 4, 64, 256, 1, None, 1, 1, 1, 16, 1, 0, None) == _lib.ERR_DTYPE  # float32 h
    assert gu(x3, 1, 1, 4, 64, 256, 1, None, 1, 1, 1, 8, 1, 1, None) == _lib.ERR_ARG  # tiles of 8
    assert gu(x3, 0, 1, 4, 64, 256, 1, None, 1, 1, 1, 16, 1, 1, None) == _lib.ERR_ARG  # null gate
    # a matrix of 4 GiB or more (row offsets within a matrix are 32-bit in these kernels)
    assert gu(x3, 1, 1, 4, 1 << 24, 4096, 1, None, 1, 1, 1, 16, 1, 1, None) == _lib.ERR_SHAPE
    dn = lib.strata_prompt_down
    assert dn(x3, 1, 4, 64, 256, 1, None, 1, 1, 16, 1, 1, -1, 1, 1, None) == _lib.ERR_ARG  # negative pairs
    assert dn(x3, 1, 4, 64, 256, 1, None, 1, 1, 16, 1, 0, 4, 1, 1, None) == _lib.ERR_ARG  # null idx
    assert dn(x3, 1, 4, 1 << 24, 4096, 1, None, 1, 1, 16, 1, 1, 4, 1, 1, None) == _lib.ERR_SHAPE  # 4 GiB matrices
    na = lib.strata_route_tiles_noalloc
    assert na(1, 65537, 8, 256, 16, 1, 1, 1, 1, None) == _lib.ERR_SHAPE  # more pairs than its array takes
    assert na(1, 4096, 8, 1025, 16, 1, 1, 1, 1, None) == _lib.ERR_SHAPE  # more experts
    assert na(1, 4096, 0, 256, 16, 1, 1, 1, 1, None) == _lib.ERR_ARG
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_SHAPE, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ERR_LAUNCH, "x")


def test_shared_expert_entry_points_check_their_arguments():
    lib = _lib.library()
    q, k4 = _lib.kind_id("IQ3_S"), _lib.kind_id("Q4_K")
    gs = lib.strata_expert_gate_up_swiglu_shared
    #        kind gate up experts rows cols idx pairs x  dtype g  u  h  s_kind s_gate s_up s_rows s_h s_g s_u stream
    assert gs(q, 1, 1, 4, 1536, 4096, 1, 8, 1, 0, 1, 1, 1, k4, 1, 1, 1536, 1, None, None, None) == _lib.ERR_DTYPE
    assert gs(q, 1, 1, 4, 1536, 4096, 1, 8, 1, 1, 1, 1, 1, q, 1, 1, 1536, 1, None, None, None) == _lib.ERR_SHAPE
    assert gs(q, 1, 1, 4, 1536, 4096, 1, 8, 1, 1, 1, 1, 1, k4, 0, 1, 1536, 1, None, None, None) == _lib.ERR_ARG
    assert gs(q, 1, 1, 4, 0, 4096, 1, 8, 1, 1, 1, 1, 1, k4, 1, 1, 1536, 1, None, None, None) == _lib.ERR_SHAPE
    assert gs(q, 1, 1, 4, 1536, 4000, 1, 8, 1, 1, 1, 1, 1, k4, 1, 1, 1536, 1, None, None, None) == _lib.ERR_SHAPE
    ms = lib.strata_expert_matvec_shared
    #        kind blocks experts rows cols idx pairs x dtype out s_kind s_blocks s_rows s_x s_out stream
    assert ms(q, 1, 4, 4096, 1536, 1, 8, 1, 0, 1, k4, 1, 4096, 1, 1, None) == _lib.ERR_DTYPE  # float32 h
    assert ms(q, 1, 4, 4096, 1536, 1, 8, 1, 1, 1, q, 1, 4096, 1, 1, None) == _lib.ERR_SHAPE  # shared not Q4_K
    assert ms(q, 1, 4, 4096, 1536, 1, 8, 1, 1, 1, k4, 1, 4096, 0, 1, None) == _lib.ERR_ARG  # null shared token
    assert ms(q, 1, 4, 4096, 1536, 1, 8, 1, 1, 1, k4, 1, 4096, 1, 0, None) == _lib.ERR_ARG  # null shared out
    assert ms(q, 1, 4, 4096, 1536, 1, 0, 1, 1, 1, k4, 1, 4096, 1, 1, None) == _lib.ERR_ARG  # no pairs
    assert ms(q, 1, 4, 0, 1536, 1, 8, 1, 1, 1, k4, 1, 4096, 1, 1, None) == _lib.ERR_SHAPE  # no routed rows
    assert ms(q, 1, 4, 4096, 1536, 1, 70000, 1, 1, 1, k4, 1, 4096, 1, 1, None) == _lib.ERR_SHAPE  # > 65535 pairs
    assert ms(q, 1, 4, 4096, 1500, 1, 8, 1, 1, 1, k4, 1, 4096, 1, 1, None) == _lib.ERR_SHAPE  # not whole blocks
    assert ms(99, 1, 4, 4096, 1536, 1, 8, 1, 1, 1, k4, 1, 4096, 1, 1, None) == _lib.ERR_KIND
    mg = lib.strata_moe_gate_up_swiglu_shared
    #        kind gate up experts rows cols logits l_rows pairs x dtype h idx w s_kind s_gate s_up s_rows s_h extra stream
    assert mg(q, 1, 1, 256, 1536, 4096, 0, 257, 8, 1, 1, 1, 1, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_ARG  # logits
    assert mg(q, 1, 1, 256, 1536, 4096, 1, 257, 8, 1, 1, 1, 0, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_ARG  # no idx
    assert mg(q, 1, 1, 256, 1536, 4096, 1, 257, 8, 1, 1, 1, 1, 0, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_ARG  # no w
    assert mg(q, 1, 1, 256, 1536, 4096, 1, 255, 8, 1, 1, 1, 1, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_SHAPE
    assert mg(q, 1, 1, 257, 1536, 4096, 1, 257, 8, 1, 1, 1, 1, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_SHAPE
    assert mg(q, 1, 1, 256, 1536, 4096, 1, 257, 65, 1, 1, 1, 1, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_SHAPE
    assert mg(q, 1, 1, 4, 1536, 4096, 1, 5, 8, 1, 1, 1, 1, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_SHAPE  # k > n
    assert mg(q, 1, 1, 256, 1536, 4096, 1, 257, 8, 1, 0, 1, 1, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_DTYPE
    assert mg(q, 1, 1, 256, 1536, 4096, 1, 257, 8, 1, 1, 1, 1, 1, q, 1, 1, 1536, 1, 1, None) == _lib.ERR_SHAPE
    assert mg(q, 1, 1, 256, 1536, 4096, 1, 257, 8, 1, 1, 0, 1, 1, k4, 1, 1, 1536, 1, 1, None) == _lib.ERR_ARG  # no h


def test_router_route_checks_its_arguments():
    lib = _lib.library()
    rr = lib.strata_router_route
    #        w rows cols x tokens dtype logits experts k idx weights extra count stream
    assert rr(1, 257, 4096, 1, 9, 1, 1, 256, 8, 1, 1, 1, 1, None) == _lib.ERR_SHAPE  # more than 8 tokens
    assert rr(1, 257, 4096, 1, 1, 1, 1, 258, 8, 1, 1, 1, 1, None) == _lib.ERR_SHAPE  # more experts than rows
    assert rr(1, 257, 4096, 1, 1, 1, 1, 256, 65, 1, 1, 1, 1, None) == _lib.ERR_SHAPE  # k past 64
    assert rr(1, 257, 4100, 1, 1, 1, 1, 256, 8, 1, 1, 1, 1, None) == _lib.ERR_SHAPE  # cols not a multiple of 8
    assert rr(1, 257, 4096, 1, 1, 2, 1, 256, 8, 1, 1, 1, 1, None) == _lib.ERR_DTYPE  # bfloat16 x
    assert rr(1, 257, 4096, 1, 1, 1, 1, 256, 8, 1, 1, 1, 0, None) == _lib.ERR_ARG  # no count
    assert rr(0, 257, 4096, 1, 1, 1, 1, 256, 8, 1, 1, 1, 1, None) == _lib.ERR_ARG  # null weights
    assert rr(1, 257, 4096, 1, 0, 1, 1, 256, 8, 1, 1, 1, 1, None) == _lib.OK  # no tokens

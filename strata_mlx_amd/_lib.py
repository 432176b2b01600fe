"""ctypes binding of libstrata_gfx950.so, the gfx950 kernels behind the C ABI in include/strata_gfx950.h.

Every device pointer is a torch tensor's `data_ptr()`; every call is enqueued on torch's current HIP
stream. A missing library raises at first use: there is no other implementation to fall back to.
"""

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libstrata_gfx950.so")

# GGUF type ids (strata_mlx/gguf.py:25-33)
KIND_IDS = {"Q4_0": 2, "Q5_0": 6, "Q8_0": 8, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ2_XXS": 16,
            "IQ2_XS": 17, "IQ3_XXS": 18, "IQ4_NL": 20, "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29,
            "Q2_0": 42}
F32, F16, BF16 = 0, 1, 2
DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
OK, ERR_KIND, ERR_SHAPE, ERR_DTYPE, ERR_LAUNCH, ERR_ARG = 0, -1, -2, -3, -4, -5
_MESSAGES = {ERR_KIND: "block type not taken by the kernels", ERR_SHAPE: "shape not taken by the kernels",
             ERR_DTYPE: "dtype not taken by the kernels", ERR_LAUNCH: "kernel launch failed",
             ERR_ARG: "invalid argument"}

# name -> (restype, argtypes); mirrors include/strata_gfx950.h
_p, _i, _i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
SIGNATURES = {
    "strata_abi_version": (_i, []),
    "strata_block_info": (_i, [_i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "strata_dequant": (_i, [_i, _p, _i64, _i64, _i64, _p, _i, _p]),
    "strata_expert_matvec": (_i, [_i, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _i64, _p, _p]),
    "strata_expert_matvec2": (_i, [_i, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _i64, _p, _p, _p]),
    "strata_router_matvec": (_i, [_p, _i64, _i64, _p, _i64, _i, _p, _p]),
    "strata_top_k": (_i, [_p, _i64, _i64, _i64, _p, _p, _p]),
    "strata_moe_combine": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i, _p, _p]),
    "strata_q2_lookup_table": (_i, [_p, _i64, _i64, _p, _p]),
    "strata_q2_lookup_table_glu": (_i, [_p, _p, _i64, _i64, _p, _p]),
    "strata_q2_lookup_matvec": (_i, [_p, _p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i, _p, _p, _p]),
    "strata_q2_lookup_down_glu": (_i, [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _i, _p, _p]),
    "strata_q3k_planes": (_i, [_p, _i64, _i64, _p, _p, _p, _p, _p]),
    "strata_q3k_planes_window": (_i, [_p, _p, _p, _p, _i64, _i64, _p, _i64, _i, _i, _p, _p]),
    "strata_q3k_planes_dequant": (_i, [_p, _p, _p, _p, _i64, _i64, _p, _i, _p]),
    "strata_expert_gate_up_swiglu": (_i, [_i, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _i64, _p, _p, _p, _p]),
    "strata_expert_gate_up_swiglu_shared": (_i, [_i, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _p, _p, _p, _i, _p,
                                                 _p, _i64, _p, _p, _p, _p]),
    "strata_expert_matvec_shared": (_i, [_i, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _p, _i, _p, _i64, _p, _p, _p]),
    "strata_router_route": (_i, [_p, _i64, _i64, _p, _i64, _i, _p, _i64, _i64, _p, _p, _p, _p, _p]),
    "strata_moe_gate_up_swiglu_shared": (_i, [_i, _p, _p, _i64, _i64, _i64, _p, _i64, _i64, _p, _i, _p, _p, _p, _i, _p,
                                              _p, _i64, _p, _p, _p]),
    "strata_expert_layer_workspace": (_i64, [_i64, _i64]),
    "strata_expert_layer": (_i, [_i, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _p, _p, _p, _i64, _p]),
    "strata_expert_matvec_swiglu": (_i, [_i, _p, _i64, _i64, _i64, _p, _i64, _p, _p, _i, _p, _p]),
    "strata_expert_matvec_ptrs": (_i, [_i, _p, _i64, _i64, _i64, _p, _i, _i64, _p, _p]),
    "strata_dense_matvec": (_i, [_i, _p, _i64, _i64, _p, _i64, _i, _p, _i, _p, _i64, _p]),
    "strata_route_tiles_max": (_i64, [_i64, _i64, _i64]),
    "strata_route_tiles_workspace": (_i64, [_i64, _i64]),
    "strata_route_tiles": (_i, [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p]),
    "strata_route_tiles_noalloc": (_i, [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p]),
    "strata_grouped_matmul": (_i, [_i, _p, _i64, _i64, _i64, _p, _i, _p, _p, _i64, _i64, _p, _p]),
    "strata_rows_to_f16": (_i, [_p, _i64, _i64, _i, _p, _p, _p]),
    "strata_rows_from_f32": (_i, [_p, _i64, _i64, _p, _i, _p, _p]),
    "strata_prompt_gate_up_swiglu": (_i, [_i, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p, _i, _p]),
    "strata_prompt_down": (_i, [_i, _p, _i64, _i64, _i64, _p, _p, _p, _i64, _i64, _p, _p, _i64, _p, _i, _p]),
}

_lib = None


def library() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (`__graft_entry__.build()` or `make -C strata_mlx_amd`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it (make -C strata_mlx_amd)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    return _lib


def check(rc: int, what: str):
    if rc == OK:
        return
    msg = f"{what}: {_MESSAGES.get(rc, f'error {rc}')}"
    if rc == ERR_LAUNCH:
        raise RuntimeError(msg)
    raise ValueError(msg)


def kind_id(kind: str) -> int:
    if kind not in KIND_IDS:
        raise ValueError(f"{kind}: not a GGUF block type")
    return KIND_IDS[kind]


def dtype_id(dtype: torch.dtype) -> int:
    if dtype not in DTYPES:
        raise ValueError(f"{dtype}: activations must be float32, float16 or bfloat16")
    return DTYPES[dtype]


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def require_device(*tensors):
    for t in tensors:
        if t is not None and (not t.is_cuda or not t.is_contiguous()):
            raise ValueError("tensors must be contiguous and on the GPU")

"""strata_mlx_amd: strata-mlx's expert dequant-matmul path, rebuilt for AMD MI355X (gfx950).

Activations multiply weights still packed in the GGUF file's block formats, through hand-written HIP
kernels behind a C ABI (include/strata_gfx950.h, libstrata_gfx950.so). The Python modules mirror the
reference's call surface with torch tensors on the GPU:

    blocks   BlockSwitchLinear, BlockSwitchGLU, dequantize, window_matvec, matvec_glu, matvec_separate,
             gate_up_swiglu, tiles_of, tile_matmul, switch_glu          (strata_mlx/blocks.py)
    dense    ScaledLinear, BlockLinear, BlockEmbedding                  (strata_mlx/dense.py)
    rows     rows_of: listed rows of an output layer, read in place     (strata_mlx/rows.py)
    fused    WindowLinear (the router), top_k, moe_combine, route,
             RoutedMoE (the MoE block)                                  (strata_mlx/fused.py)
    gguf     GGUF, shards, upload, experts, linear, embedding           (strata_mlx/gguf.py, load.py)
    synth    synthetic blocks and Zipf routing for benchmarks and tests
"""

__all__ = ["blocks", "dense", "rows", "fused", "gguf", "synth"]

/* strata_gfx950: the expert dequant-matmul path of strata-mlx, for AMD MI355X (gfx950).
 *
 * Activations multiply weights still packed in the GGUF file's own block formats. A block type is
 * given by its GGUF type id (strata_mlx/gguf.py:25-33): Q4_0 2, Q5_0 6, Q8_0 8, Q3_K 11, Q4_K 12, Q5_K 13,
 * Q6_K 14, IQ3_XXS 18, IQ4_NL 20, IQ3_S 21, IQ4_XS 23, Q2_0 42. A stack of matrices is laid out as
 * the file lays it out: row r of matrix e starts at byte (e * rows + r) * row_bytes, where
 * row_bytes = cols / weights_per_block * bytes_per_block.
 *
 * Every pointer is a device pointer (so is each of strata_expert_matvec_ptrs's per_pair), and every
 * call only enqueues work on `stream` (a hipStream_t; NULL is the default stream). The library
 * allocates nothing and never waits for the device. The caller owns all memory: inputs are only read and
 * outputs are fully written. Calls are reentrant across host threads and streams.
 * Activation/output dtypes: STRATA_F32, STRATA_F16, STRATA_BF16. Sums are float32 throughout.
 *
 * Each entry point returns STRATA_OK (0) or a negative STRATA_ERR_* code: the Python layer raises
 * ValueError for KIND / SHAPE / DTYPE / ARG, as the reference does for a type or shape its kernels
 * do not take (strata_mlx/blocks.py:294-295, dense.py:118-119), and RuntimeError for LAUNCH.
 */
#ifndef STRATA_GFX950_H
#define STRATA_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { STRATA_F32 = 0, STRATA_F16 = 1, STRATA_BF16 = 2 };
enum {
  STRATA_OK = 0,
  STRATA_ERR_KIND = -1,   /* a block type the kernels do not decode */
  STRATA_ERR_SHAPE = -2,  /* rows of cols weights do not end on a block, or a size out of range */
  STRATA_ERR_DTYPE = -3,  /* an activation/output dtype the call does not take */
  STRATA_ERR_LAUNCH = -4, /* the HIP launch failed */
  STRATA_ERR_ARG = -5     /* a null pointer or a count out of range */
};

/* ABI version of this header. */
int strata_abi_version(void);

/* Weights and bytes per block of `kind`; STRATA_ERR_KIND if the kernels do not decode it.
 * Replaces the BLOCK table, strata_mlx/blocks.py:36-38. */
int strata_block_info(int kind, int* per_block, int* block_bytes);

/* out[m, r, c] = the weight (m, r, c) of `n_mats` matrices of rows x cols, as float32/16 (bit-exact:
 * each weight is computed exactly in float32 and rounded once to out_dtype).
 * Replaces dequantize + _DEQUANT, strata_mlx/blocks.py:515-522, 261-270. */
int strata_dequant(int kind, const void* blocks, int64_t n_mats, int64_t rows, int64_t cols, void* out,
                   int out_dtype, void* stream);

/* out[p, r] = W[idx[p], r, :] . x[p / share, :] for p < pairs, W a stack of `experts` matrices of
 * rows x cols; out (pairs, rows) in x's dtype. Pairs that name the same expert read its bytes once.
 * A pair naming no expert (idx >= experts) gets NaN rows; experts must be at least 1 when pairs > 0.
 * Replaces BlockSwitchLinear.__call__ + _MATVEC, strata_mlx/blocks.py:538-554, 196-220. */
int strata_expert_matvec(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                         const uint32_t* idx, int64_t pairs, const void* x, int x_dtype, int64_t share,
                         void* out, void* stream);

/* strata_expert_matvec over two stacks of one shape that read the same x (gate and up), one launch.
 * Replaces the gate and up calls of switch_glu, strata_mlx/blocks.py:969. */
int strata_expert_matvec2(int kind, const void* blocks_a, const void* blocks_b, int64_t experts, int64_t rows,
                          int64_t cols, const uint32_t* idx, int64_t pairs, const void* x, int x_dtype,
                          int64_t share, void* out_a, void* out_b, void* stream);

/* strata_expert_matvec2 over the gate and up stacks that also writes out_h = swiglu(out_gate, out_up)
 * rounded as strata_expert_matvec_swiglu rounds it; out_gate, out_up, out_h (pairs, rows). The float16
 * IQ3_S / IQ3_XXS / Q2_0 kernels do it in the one launch (a lane holds both sums of a row); others add a
 * small elementwise launch. Replaces the gate and up calls of switch_glu and the swiglu of its down call,
 * strata_mlx/blocks.py:969-975 with _MATVEC_GLU's rounding, strata_mlx/blocks.py:222-236. */
int strata_expert_gate_up_swiglu(int kind, const void* gate_blocks, const void* up_blocks, int64_t experts,
                                 int64_t rows, int64_t cols, const uint32_t* idx, int64_t pairs, const void* x,
                                 int x_dtype, int64_t share, void* out_gate, void* out_up, void* out_h,
                                 void* stream);

/* strata_expert_gate_up_swiglu at one token (every pair reads x's one row) with a shared expert's gate and up
 * in the same launch: shared_h[r] = silu(shared_gate[r, :] . x) * (shared_up[r, :] . x), rounded as out_h;
 * shared_gate, shared_up (shared_rows, cols); shared_g and shared_u (each NULL or (shared_rows,)) get the shared
 * expert's gate . x and up . x as float16. The routed stacks IQ3_S or Q2_0 of 4096 inputs, x float16, the
 * shared expert Q4_K; other cases return STRATA_ERR_SHAPE, and the caller makes the two calls apart. No single
 * counterpart in the reference, whose MoE block calls the routed experts and then the shared expert
 * (strata_mlx/fused.py:492-493, the gate and up of each, with the SwiGLU of their down calls): the routed
 * launch's waves take the shared expert's rows among their own, which spares its own launch. */
int strata_expert_gate_up_swiglu_shared(int kind, const void* gate_blocks, const void* up_blocks, int64_t experts,
                                        int64_t rows, int64_t cols, const uint32_t* idx, int64_t pairs,
                                        const void* x, int x_dtype, void* out_gate, void* out_up, void* out_h,
                                        int shared_kind, const void* shared_gate, const void* shared_up,
                                        int64_t shared_rows, void* shared_h, void* shared_g, void* shared_u,
                                        void* stream);

/* strata_expert_gate_up_swiglu_shared with the pairs' experts chosen in the launch: logits (logit_rows float32,
 * the router's products for one token: the `experts` experts' first, then any rows past them, such as a shared
 * expert's gate), pairs = k, the top k of the experts' logits and their softmax (as strata_top_k chooses them:
 * ties to the lower index) written to idx_out (k) and w_out (k) for the down and combine calls, and the rows past
 * the experts' rounded to float16 into extra_out (logit_rows - experts, or NULL). out_h and shared_h as
 * strata_expert_gate_up_swiglu_shared gives them; a logit that is NaN is never chosen, and a pair left without an
 * expert gets index 0xffffffff and NaN in out_h. experts <= 256, k <= 64; the routed stacks IQ3_S or Q2_0 of 4096
 * inputs at three units a wave (on 256 CUs, IQ3_S 3 to 8 pairs of 1536 rows, Q2_0 6 to 8); other cases return
 * STRATA_ERR_SHAPE (the choice then from strata_router_route). No counterpart in the reference, whose MoE block calls the router, top_k and the
 * experts apart (strata_mlx/fused.py:488-493): the launch's workgroups make the choice while their codebooks
 * fill, which spares the router's launch its choice. */
int strata_moe_gate_up_swiglu_shared(int kind, const void* gate_blocks, const void* up_blocks, int64_t experts,
                                     int64_t rows, int64_t cols, const float* logits, int64_t logit_rows,
                                     int64_t pairs, const void* x, int x_dtype, void* out_h, uint32_t* idx_out,
                                     float* w_out, int shared_kind, const void* shared_gate, const void* shared_up,
                                     int64_t shared_rows, void* shared_h, void* extra_out, void* stream);

/* strata_expert_matvec at one token (each pair's own x, share 1: the down call of a routed layer) with a shared
 * expert's down in the same launch: shared_out[r] = shared_blocks[r, :] . shared_x, shared_blocks a Q4_K matrix of
 * shared_rows x cols, shared_x its token (float16, its h), shared_out float16. The routed stack IQ3_S or Q2_0 of
 * 1536 inputs, x float16; out gets strata_expert_matvec's bits. The launch has pairs * ceil(rows / 128)
 * workgroups, and each takes 16 of the shared rows: more shared rows than that, another kind or width, or a
 * routed case that runs faster at two units a wave return STRATA_ERR_SHAPE, and the caller then makes the two
 * calls apart. No counterpart in the reference, whose MoE block calls the routed
 * experts and then the shared expert (strata_mlx/fused.py:492-493, each down with its SwiGLU): the routed down
 * launch's waves take the shared expert's rows among their own, which spares its own launch. */
int strata_expert_matvec_shared(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                                const uint32_t* idx, int64_t pairs, const void* x, int x_dtype, void* out,
                                int shared_kind, const void* shared_blocks, int64_t shared_rows, const void* shared_x,
                                void* shared_out, void* stream);

/* The routed experts of one decode token in one launch: h[p, :] = swiglu(gate[idx[p]] . x, up[idx[p]] . x) rounded
 * as strata_expert_gate_up_swiglu rounds it, then out[p, :] = down[idx[p]] . h[p, :]; the same bits as those two
 * calls (strata_expert_gate_up_swiglu, then strata_expert_matvec on down). gate, up (experts, ffn, hidden) and down
 * (experts, hidden, ffn) stacks of `kind` IQ3_S or Q2_0, hidden 4096, ffn 1536 or 2560; x one float16 token;
 * pairs 1 to 16 (ffn 2560: 1 to 8 on a 256-CU part; more return STRATA_ERR_SHAPE and the caller makes the two
 * calls); out (pairs, hidden) float16; out_h (pairs, ffn) float16 or NULL. A pair naming no expert gets NaN rows.
 * `workspace`: device memory of strata_expert_layer_workspace(pairs, ffn) bytes for the largest (pairs, ffn) it
 * serves, zeroed before its first call; calls of any shape on one device may then share it one after another
 * (every call advances every workgroup's launch count; calls that share a workspace must not overlap). One
 * workgroup a CU runs for the launch and the workgroups of a pair wait for each other's h:
 * each wait gives up after `spin` polls of memory (about a microsecond each; 100000 is ample), writes NaN to its
 * rows of out and sets bit 0 of the workspace's first uint32, which the caller reads and clears. Replaces the
 * per-pair path of switch_glu at one token, strata_mlx/blocks.py:958-986 (the gate and up calls, then matvec_glu's
 * down with the SwiGLU, :939-955). */
int64_t strata_expert_layer_workspace(int64_t pairs, int64_t ffn);
int strata_expert_layer(int kind, const void* gate_blocks, const void* up_blocks, const void* down_blocks,
                        int64_t experts, int64_t hidden, int64_t ffn, const uint32_t* idx, int64_t pairs,
                        const void* x, int x_dtype, void* out_h, void* out, void* workspace, int64_t spin,
                        void* stream);

/* out[p, r] = W[idx[p], r, :] . swiglu(gate[p], up[p]) with the SwiGLU rounded as mlx-lm rounds it
 * (sigmoid in float32 rounded to the activation dtype, then two products in that dtype); gate, up
 * (pairs, cols). Replaces matvec_glu + _MATVEC_GLU, strata_mlx/blocks.py:939-955, 225-259. */
int strata_expert_matvec_swiglu(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                                const uint32_t* idx, int64_t pairs, const void* gate, const void* up,
                                int act_dtype, void* out, void* stream);

/* out[p, r] = E_p[r, :] . x[p / share, :] where per_pair[p] (a device array of device pointers) is
 * pair p's own rows x cols matrix. Replaces matvec_separate, strata_mlx/blocks.py:331-346. */
int strata_expert_matvec_ptrs(int kind, const void* const* per_pair, int64_t rows, int64_t cols, int64_t pairs,
                              const void* x, int x_dtype, int64_t share, void* out, void* stream);

/* out[t, j] = W[row(j), :] . x[t, :] for one matrix W (rows x cols) and `tokens` rows of x; row(j) =
 * row_ids[j] for j < n_ids when row_ids is given (a device array), else j < rows. out (tokens, n)
 * in out_dtype. A token gets the same bits whatever the number of tokens with it.
 * Replaces window_matvec (strata_mlx/blocks.py:383-394), ScaledLinear on Q6_K blocks
 * (strata_mlx/dense.py:141-167), BlockLinear (dense.py:224-242) and _rows_of (strata_mlx/rows.py:30-42). */
int strata_dense_matvec(int kind, const void* blocks, int64_t rows, int64_t cols, const void* x, int64_t tokens,
                        int x_dtype, void* out, int out_dtype, const uint32_t* row_ids, int64_t n_ids,
                        void* stream);

/* Tiles a prompt's pairs can need at most: pairs / tile + min(experts, pairs). */
int64_t strata_route_tiles_max(int64_t pairs, int64_t experts, int64_t tile);

/* The pairs idx (tokens x k, flattened) laid out in tiles of `tile` slots, each tile one expert's,
 * on the device with no host wait: tile_expert[n_tiles] (`experts` for a tile nothing fills),
 * token[n_tiles * tile] (0 for an empty slot), where[pairs] (the slot of each pair) and, if not
 * NULL, slot_pair[n_tiles * tile] (the pair of each slot, 0xffffffff for an empty one), with
 * n_tiles = strata_route_tiles_max(pairs, experts, tile). Slots of an expert go in pair order. A pair
 * naming no expert (>= experts) gets no slot: its `where` is 0xffffffff. `workspace` is device memory of
 * strata_route_tiles_workspace(pairs, experts) bytes. Replaces tiles_of, strata_mlx/blocks.py:657-681. */
int64_t strata_route_tiles_workspace(int64_t pairs, int64_t experts);
int strata_route_tiles(const uint32_t* idx, int64_t pairs, int64_t k, int64_t experts, int64_t tile,
                       uint32_t* tile_expert, uint32_t* token, uint32_t* where, uint32_t* slot_pair,
                       void* workspace, void* stream);

/* 16-bit rows scaled into float16 by a power of two, for the MFMA kernels below: out[r, c] = a[r, c] / 2^e(r),
 * e(r) = floor(log2 m(r)) - 14 with m(r) = max_c |a[r, c]| (e = 0 for a row of zeros or one holding an infinity or
 * NaN), so each row's largest magnitude lands in [2^14, 2^15); row_max[r] = the float bits of m(r). Every value
 * within 2^31 of m(r) is exact in float16 (all of a bfloat16 row whose values span fewer than 31 binades); smaller
 * ones round to float16's subnormal steps, an error below 2^-39 m(r). a_dtype BF16, F16 or F32; out float16
 * (rows, cols). No counterpart in the reference, whose tile kernel takes float16 and float32 only
 * (strata_mlx/blocks.py:960): this is how bfloat16 activations reach the float16 MFMA exactly. */
int strata_rows_to_f16(const void* a, int64_t rows, int64_t cols, int a_dtype, void* out, uint32_t* row_max,
                       void* stream);

/* The inverse of strata_rows_to_f16's scaling, for products of the scaled rows: out[r, c] = c[r, c] * 2^e(r) rounded
 * once to out_dtype (BF16, F16 or F32), e(r) from row_max[r] as strata_rows_to_f16 set it; c float32 (rows, cols),
 * out (rows, cols), at most 65535 rows. No counterpart in the reference, which multiplies a prompt chunk's
 * bfloat16 tokens by weights in bfloat16 (strata_mlx/dense.py:234-241): here the tokens are scaled into float16
 * exactly, multiplied by float16 weights with float32 sums, and their sums come back through this call. */
int strata_rows_from_f32(const float* c, int64_t rows, int64_t cols, const uint32_t* row_max, int out_dtype,
                         void* out, void* stream);

/* strata_route_tiles with its workspace in the library's own device memory (a file-scope array of about 1 MB a
 * GPU, held until the process ends): the call allocates nothing, for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. pairs at
 * most 65536 and experts at most 1024, else STRATA_ERR_SHAPE; STRATA_ERR_LAUNCH if the array's address cannot be
 * found. The first call on a device looks that address up (with that device current). Every call on one GPU uses
 * the same array: calls that overlap on one GPU (two streams, two threads) race. The outputs are those of
 * strata_route_tiles, bit for bit. */
int strata_route_tiles_noalloc(const uint32_t* idx, int64_t pairs, int64_t k, int64_t experts, int64_t tile,
                               uint32_t* tile_expert, uint32_t* token, uint32_t* where, uint32_t* slot_pair,
                               void* stream);

/* c[s, :] = W[tile_expert[s / tile]] . a[s, :] for s < n_tiles * tile; a (n_tiles * tile, cols) in
 * a_dtype (F16 or F32), c (n_tiles * tile, rows) float32. Tiles naming no expert (>= experts) are skipped and
 * their rows of c are left as they were. a_max (F16 only, or NULL): a's rows were scaled by strata_rows_to_f16
 * and a_max is its row_max; the sums are scaled back exactly. F16 activations go to MFMA as they are (float32
 * sums): IQ3_S / IQ3_XXS / Q2_0 rows of whole 256-weight steps multiply exact weights (integer codes times the
 * run's own scale, exact in float16, with d on the float32 sums; Q2_0 exact while |d| <= 32752), other types
 * weights rounded to float16. F32 activations multiply exact weights in float32.
 * Replaces tile_matmul + _TILES, strata_mlx/blocks.py:634-654, 583-626. */
int strata_grouped_matmul(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols,
                          const void* a, int a_dtype, const uint32_t* a_max, const uint32_t* tile_expert,
                          int64_t n_tiles, int64_t tile, float* c, void* stream);

/* The gate and up products of a prompt's tiles and the SwiGLU between them, in one launch: for every slot s of a
 * tile naming an expert e(s) < experts, h[s, r] = silu(g) * u rounded once to h_dtype (F16 or BF16) from float32,
 * g = G[e(s)][r] . x[token[s]], u = U[e(s)][r] . x[token[s]] (float32 sums; silu(g) * u as mlx-lm's swiglu
 * computes it on float32 products). x float16 (tokens, cols): as given, or scaled by strata_rows_to_f16 with x_max
 * its row_max (else NULL). gate / up (experts, rows, cols) stacks; h (n_tiles * tile, rows); token as
 * strata_route_tiles gives it. Tiles naming no expert leave their rows of h as they were. IQ3_S / IQ3_XXS / Q2_0
 * stacks with cols a multiple of 256, else STRATA_ERR_KIND (the caller takes strata_grouped_matmul twice).
 * Replaces the gate and up tile products and the swiglu of _tiled_glu, strata_mlx/blocks.py:684-692. */
int strata_prompt_gate_up_swiglu(int kind, const void* gate, const void* up, int64_t experts, int64_t rows,
                                 int64_t cols, const void* x, const uint32_t* x_max, const uint32_t* token,
                                 const uint32_t* tile_expert, int64_t n_tiles, int64_t tile, void* h, int h_dtype,
                                 void* stream);

/* The down product of a prompt's tiles written to the pairs: y[slot_pair[s], r] = W[e(s)][r] . h[s] rounded once
 * to y_dtype (F16 or BF16) from the float32 sum, for every slot s of a tile naming an expert and holding a pair;
 * y[p, :] = NaN for the pairs p naming no expert (idx[p] >= experts, idx the pairs' experts). h float16
 * (n_tiles * tile, cols) in slot order, as given or scaled (h_max its row_max, else NULL); y (pairs, rows);
 * slot_pair as strata_route_tiles gives it. Kinds and shapes as strata_prompt_gate_up_swiglu.
 * Replaces the down tile product and the [where] gather of _tiled_glu, strata_mlx/blocks.py:693-694. */
int strata_prompt_down(int kind, const void* blocks, int64_t experts, int64_t rows, int64_t cols, const void* h,
                       const uint32_t* h_max, const uint32_t* tile_expert, int64_t n_tiles, int64_t tile,
                       const uint32_t* slot_pair, const uint32_t* idx, int64_t pairs, void* y, int y_dtype,
                       void* stream);

/* out[t, r] = W[r, :] . x[t, :] for a float16 W (rows x cols, row-major) and `tokens` rows of x
 * (STRATA_F16 or STRATA_F32); out (tokens, rows) float32. cols must be a multiple of 8. The router's
 * product, read as the weights are. Replaces WindowLinear + _MATVEC, strata_mlx/fused.py:334-390. */
int strata_router_matvec(const void* w, int64_t rows, int64_t cols, const void* x, int64_t tokens, int x_dtype,
                         float* out, void* stream);

/* idx[r, :] = the k largest of logits[r, :] (rows x n float32), largest first, ties to the lower index
 * (what a stable sort gives); if `weights` is not NULL, weights[r, :] = the softmax of those k logits
 * (float32). n <= 2048, k <= 64. Replaces top_k + _TOPK and the softmax of _Routed.__call__,
 * strata_mlx/fused.py:400-436, 490-491. */
int strata_top_k(const float* logits, int64_t rows, int64_t n, int64_t k, uint32_t* idx, float* weights,
                 void* stream);

/* strata_router_matvec and strata_top_k in one launch, at 1-8 tokens: logits (tokens, rows) float32 = W . x as
 * strata_router_matvec gives them; idx (tokens, k) and weights (tokens, k, or NULL) as strata_top_k gives them
 * over each token's first `experts` logits (experts <= 2048, k <= 64); extra (tokens, rows - experts) float16, or
 * NULL: the rows past the experts' rounded once (a shared expert's gate, one more row of W). `count` is a uint32
 * of device memory, zero before the first call, that the launch leaves at zero: the workgroups count themselves
 * there, and the last to finish its rows makes the choice. Calls that overlap on one `count` race: one a stream.
 * No single counterpart in the reference, whose MoE block calls the router, top_k and the shared expert's gate
 * apart (WindowLinear + _MATVEC, top_k + _TOPK, the softmax and shared_expert_gate of _Routed.__call__,
 * strata_mlx/fused.py:356-390, 400-436, 488-493); tokens past 8 return STRATA_ERR_SHAPE (those calls apart). */
int strata_router_route(const void* w, int64_t rows, int64_t cols, const void* x, int64_t tokens, int x_dtype,
                        float* logits, int64_t experts, int64_t k, uint32_t* idx, float* weights, void* extra,
                        uint32_t* count, void* stream);

/* out[t, :] = half(sum_j y[t, j, :] * w[t, j]) + half(half(sigmoid(g[t])) * s[t, :]): y (rows, k, d),
 * g (rows), s and out (rows, d) float16, w (rows, k) float32. The experts are added in the order of the
 * reference (eight partial sums, expert j into sum j % 8, each product rounded before it is added, then
 * the sums in order); each float16 operation rounds once. Replaces moe_combine + _COMBINE,
 * strata_mlx/fused.py:448-481. */
int strata_moe_combine(const void* y, const float* w, const void* g, const void* s, int64_t rows, int64_t k,
                       int64_t d, int dtype, void* out, void* stream);

/* The Q2_0 table of sums (float16 only). table (tokens, cols / 2, 16) float16: entry c of input pair g of token
 * t is (c & 3 - 1) * x[t, 2g] + (c >> 2 - 1) * x[t, 2g + 1], summed in float32 and rounded once. Replaces
 * lookup_table + _TABLE, strata_mlx/blocks.py:718-781. */
int strata_q2_lookup_table(const void* x, int64_t tokens, int64_t cols, void* table, void* stream);

/* The same table of silu(gate) * up (sigmoid in float32 with expf, nothing rounded before the sums). Replaces
 * lookup_table_glu + _TABLE_GLU, strata_mlx/blocks.py:728-795. */
int strata_q2_lookup_table_glu(const void* gate, const void* up, int64_t tokens, int64_t cols, void* table,
                               void* stream);

/* out[p, r] = W[idx[p], r, :] . x[p / share] for a Q2_0 stack, x given as its table; float16 out (pairs, rows).
 * per_row lanes a row (a power of two <= 32): lane `part` sums runs part, part + per_row, ... and the row's
 * total is their sums in lane order, so per_row fixes the bits. With blocks_b / out_b (not NULL), a second stack
 * of the same shape in the same launch, each row summed as alone (gate and up). cols <= 4096, a multiple of 64.
 * Replaces lookup_matvec + _LOOKUP and lookup_gate_up + _LOOKUP_TWO, strata_mlx/blocks.py:741-761, 798-852. */
int strata_q2_lookup_matvec(const void* blocks, const void* blocks_b, int64_t experts, int64_t rows, int64_t cols,
                            const uint32_t* idx, int64_t pairs, const void* table, int64_t share, int per_row,
                            void* out, void* out_b, void* stream);

/* strata_q2_lookup_matvec(..., table of strata_q2_lookup_table_glu(gate, up), share 1) in one launch, each pair's
 * table built in LDS: the same bits. gate, up (pairs, cols) float16. Replaces lookup_down_glu + _DOWN_GLU,
 * strata_mlx/blocks.py:855-914. */
int strata_q2_lookup_down_glu(const void* blocks, int64_t experts, int64_t rows, int64_t cols, const uint32_t* idx,
                              int64_t pairs, const void* gate, const void* up, int per_row, void* out, void* stream);

/* Q3_K held as planes: a (rows, cols) Q3_K tensor's blocks rearranged once into hm (blocks x 8 uint32: the 32
 * high-bit bytes), qs (blocks x 16 uint32: the 64 value bytes), sc (blocks x 16 int8: the 6-bit scales decoded,
 * less 32) and dd (blocks float16: d), blocks = rows * cols / 256. Replaces q3k_planes,
 * strata_mlx/blocks.py:397-414. */
int strata_q3k_planes(const void* blocks, int64_t rows, int64_t cols, uint32_t* hm, uint32_t* qs, int8_t* sc,
                      void* dd, void* stream);

/* out[t, r] = W[r, :] . x[t, :] for up to 8 tokens of x (STRATA_F32 / F16 / BF16; at most 48 KB of them), W as
 * planes; out (tokens, rows) in x's type. per_row lanes a row (a power of two <= 64) fix the sums' order: chosen by the tensor's shape,
 * a token gets the same bits alone as in a window. Replaces q3k_planes_window + _Q3K_PLANES_WINDOW,
 * strata_mlx/blocks.py:425-501. */
int strata_q3k_planes_window(const uint32_t* hm, const uint32_t* qs, const int8_t* sc, const void* dd, int64_t rows,
                             int64_t cols, const void* x, int64_t tokens, int x_dtype, int per_row, void* out,
                             void* stream);

/* Every weight of a tensor held as planes, (rows, cols) float32 / float16, bit-exact. Replaces
 * q3k_planes_dequantize + _Q3K_PLANES_DEQUANT, strata_mlx/blocks.py:464-512. */
int strata_q3k_planes_dequant(const uint32_t* hm, const uint32_t* qs, const int8_t* sc, const void* dd, int64_t rows,
                              int64_t cols, void* out, int out_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRATA_GFX950_H */

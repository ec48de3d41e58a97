/* strata_hip.h — the C ABI of libstrata_hip.so: strata-mlx's decode-step hot path on MI355X (gfx950).
 *
 * Conventions
 *   - Every pointer is device memory the caller owns (e.g. a torch tensor's data_ptr()), except where noted.
 *   - `stream` is a hipStream_t (NULL: the default stream). Calls only enqueue work; they return at once.
 *   - Return 0 on success, a negative status on error (SH_E_*); sh_last_error() gives the calling thread's message.
 *     No C++ exception crosses the ABI. Shape and pointer errors are found before anything is launched.
 *   - Blocks are a tensor's GGUF bytes as the file has them; a stack of experts is experts x rows x row_bytes.
 *   - `tables` is the codebook blob (sh_tables_bytes() bytes, layout in csrc/common.h) for the kinds that read
 *     a codebook (IQ4_*, IQ3_*, IQ2_*, IQ1_M); it may be NULL for Q2_0 and Q3_K.
 *   - Expert indices that name no expert (< 0 or >= experts) give zero outputs instead of reading out of bounds.
 *
 * Each entry point names the reference interface it replaces (paths relative to the strata-mlx repository).
 */
#ifndef STRATA_HIP_H
#define STRATA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* block kinds: strata_mlx/blocks.py:36-38 (BLOCK) */
#define SH_KIND_Q2_0 0
#define SH_KIND_IQ4_NL 1
#define SH_KIND_IQ4_XS 2
#define SH_KIND_IQ3_S 3
#define SH_KIND_IQ3_XXS 4
#define SH_KIND_IQ2_S 5
#define SH_KIND_IQ2_XS 6
#define SH_KIND_IQ2_XXS 7
#define SH_KIND_IQ1_M 8
#define SH_KIND_Q3_K 9

/* activation / output element types */
#define SH_DTYPE_F32 0
#define SH_DTYPE_F16 1
#define SH_DTYPE_BF16 2

/* statuses */
#define SH_OK 0
#define SH_E_ARG (-1)
#define SH_E_SHAPE (-2)
#define SH_E_KIND (-3)
#define SH_E_DTYPE (-4)
#define SH_E_HIP (-5)
#define SH_E_WORKSPACE (-6)
#define SH_E_UNSUPPORTED (-7)

int sh_version(void);
const char* sh_last_error(void);
/* strata_mlx/blocks.py:36-38 (BLOCK): weights and bytes of a block of `kind` (host pointers). */
int sh_kind_block(int kind, int* weights_per_block, int* bytes_per_block);
/* strata_mlx/blocks.py:272-289 (_table): bytes of the codebook blob the kernels read. */
size_t sh_tables_bytes(void);

/* strata_mlx/blocks.py:397-404 (dequantize) and 261-270 (_DEQUANT): every weight of n_mats (rows x cols)
 * matrices, out_dtype F32 (exact), F16 or BF16 (one rounding). Coalesced 16-byte loads and stores where the blocks
 * and the output are 16-byte aligned and an output row fits 32 KiB, else a run a thread: the same values. */
int sh_dequantize(int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows, int64_t cols,
                  void* out, int out_dtype, void* stream);

/* strata_mlx/blocks.py:407-436 (BlockSwitchLinear.__call__, kernel _MATVEC 196-220):
 * out[pair, r] = W[idx[pair], r, :] . x[pair / share, :], out in x's dtype. bf16/fp16 activations of Q2_0 and
 * IQ3_S take the MFMA path, everything else exact float32 weights and sums (the exact-weight stream over the
 * pairs where it takes them: blocks and x 16-byte aligned). Pairs sharing an expert read its blocks once (MFMA
 * path). `workspace` may be NULL when sh_switch_workspace() is 0. */
size_t sh_switch_workspace(int kind, int64_t rows, int64_t cols, int64_t pairs, int x_dtype);
int sh_switch_matvec(int kind, const void* blocks, const void* tables, int64_t experts, int64_t rows, int64_t cols,
                     const int32_t* idx, int64_t pairs, const void* x, int x_dtype, int64_t share, void* out,
                     void* workspace, size_t workspace_bytes, void* stream);
/* the same product with exact float32 weights and sums for every kind and dtype (no MFMA); `expert_ptrs`
 * (device array of per-pair block pointers, each inside an allocation that starts on 16 bytes) replaces blocks +
 * idx when not NULL. The exact-weight stream where it takes the pairs (x 16-byte aligned), else a block a few rows
 * a pair. */
int sh_switch_matvec_generic(int kind, const void* blocks, const void* const* expert_ptrs, const void* tables,
                             int64_t experts, int64_t rows, int64_t cols, const int32_t* idx, int64_t pairs,
                             const void* x, int x_dtype, int64_t share, void* out, void* stream);

/* strata_mlx/blocks.py:351-394 (window_matvec) over a stack: out[m][t] = W_m . x[m][t], x (n_mats, tokens, cols),
 * out (n_mats, tokens, rows) in x's type. Q2_0 or IQ3_S with bf16 / fp16 activations, cols a multiple of 256 up
 * to 4096 (wider rows where the waves' column splits and the LDS ring allow: sh_stack_takes says), up to 16 tokens:
 * the MFMA kernels. Every other kind, and float32 activations: the exact-weight stream (float32 sums; the bits of
 * sh_switch_matvec_generic for the codebook kinds; Q2_0, IQ4_NL, IQ4_XS and Q3_K with their scales taken out of
 * each run's sums), up to 8 tokens whose activations fit 96 KiB of LDS, blocks and x 16-byte aligned.
 * One streaming launch over all matrices (one per window of row tiles for the longest Q2_0 stacks).
 * workspace: sh_stack_workspace() bytes (none). */
size_t sh_stack_workspace(int kind, int64_t n_mats, int64_t rows, int64_t cols, int64_t tokens, int x_dtype);
int sh_stack_matvec(int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows, int64_t cols,
                    const void* x, int x_dtype, int64_t tokens, void* out, void* workspace, size_t workspace_bytes,
                    void* stream);
/* No counterpart in the reference, whose window matvec (strata_mlx/blocks.py:351-394) takes rows of every width:
 * 1 if sh_stack_matvec takes these arguments, 0 if it refuses them (its checks and launch plan, nothing launched),
 * for a caller choosing between it and sh_window_matvec. */
int sh_stack_takes(int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows, int64_t cols,
                   const void* x, int x_dtype, int64_t tokens);

/* strata_mlx/blocks.py:331-346 (matvec_separate): one expert buffer per pair, `expert_ptrs` a device array of
 * `pairs` pointers. */
int sh_matvec_separate(int kind, const void* const* expert_ptrs, const void* tables, int64_t rows, int64_t cols,
                       int64_t pairs, const void* x, int x_dtype, int64_t share, void* out, void* stream);

/* strata_mlx/blocks.py:351-394 (window_matvec): out[t] = W . x[t], one layer, tokens <= 8; exact weights and
 * float32 sums (the exact-weight stream where it takes the layer, the bits of sh_stack_matvec's; else a block a few
 * rows). */
int sh_window_matvec(int kind, const void* blocks, const void* tables, int64_t rows, int64_t cols, const void* x,
                     int x_dtype, int64_t tokens, void* out, void* stream);

/* strata_mlx/blocks.py:782-798 (matvec_glu, kernel _MATVEC_GLU 225-259): out[pair] = W[idx[pair]] .
 * swiglu(gate[pair], up[pair]) with the reference's roundings; dtype F32, F16 or BF16 for gate, up and out. */
int sh_matvec_glu(int kind, const void* blocks, const void* tables, int64_t experts, int64_t rows, int64_t cols,
                  const int32_t* idx, int64_t pairs, const void* gate, const void* up, int dtype, void* out,
                  void* stream);

/* Q2_0 table of sums: strata_mlx/blocks.py:650-659 (lookup_table), 662-671 (lookup_table_glu), 674-695
 * (lookup_matvec), 740-760 (lookup_down_glu). Tables are (n, cols / 2, 16) in `dtype`. */
int sh_lookup_table(const void* x, int dtype, int64_t n, int64_t cols, void* table, void* stream);
int sh_lookup_table_glu(const void* gate, const void* up, int dtype, int64_t n, int64_t cols, void* table,
                        void* stream);
int sh_lookup_matvec(const void* blocks, int64_t experts, int64_t rows, int64_t cols, const int32_t* idx,
                     int64_t pairs, const void* table, int dtype, int64_t share, void* out, void* stream);
int sh_lookup_down_glu(const void* blocks, int64_t experts, int64_t rows, int64_t cols, const int32_t* idx,
                       int64_t pairs, const void* gate, const void* up, int dtype, void* out, void* stream);

/* strata_mlx/fused.py:357-390 (WindowLinear): fp16/bf16 W (rows x cols) times x (tokens <= 8) -> float32. */
int sh_router_matvec(const void* w, int w_dtype, int64_t rows, int64_t cols, const void* x, int x_dtype,
                     int64_t tokens, float* out, void* stream);

/* strata_mlx/fused.py:281-323 (FusedResidual.__call__; kernels _NORM, _DOWN, _UP at 46-131): the hyper-connection
 * read of a window of tokens <= 16 with the write before it. before (tokens x hc * d), out (tokens x d), inject_in
 * (tokens x hc) in `dtype` (F32 / F16 / BF16); norm float32 (hc * d); down (rank x hc * d), up (hc * d x rank),
 * inject_w (n_inject x hc * d, n_inject 0 or hc) in `w_dtype`, 16-byte aligned. Writes residual (tokens x hc * d:
 * before + out * inject_in), mixed (tokens x d: the block's input) and, with inject rows, inject (tokens x hc: 2
 * sigmoid of the inject rows' gate); sums in float32. hc 1, 2, 4 or 8; d a multiple of 64; rank 32..512 a
 * multiple of 32. workspace: sh_hc_workspace() bytes. */
size_t sh_hc_workspace(int64_t tokens, int64_t hc, int64_t d, int64_t rank, int64_t n_inject);
int sh_hc_residual(const void* before, const void* out, const void* inject_in, int dtype, const void* norm,
                   const void* down, const void* up, const void* inject_w, int w_dtype, int64_t tokens, int64_t hc,
                   int64_t d, int64_t rank, int64_t n_inject, float eps, void* residual, void* mixed, void* inject,
                   void* workspace, size_t workspace_bytes, void* stream);

/* strata_mlx/fused.py:424-436 (top_k, kernel _TOPK 400-418) and 491 (softmax of the chosen logits):
 * idx (rows x k) of the k largest, largest first, ties to the lower index; weights (nullable) float32. */
int sh_top_k(const void* logits, int dtype, int64_t rows, int64_t n, int64_t k, int32_t* idx, float* weights,
             void* stream);

/* strata_mlx/fused.py:467-481 (moe_combine, kernel _COMBINE 448-462): out = OutT(sum_k y_k w_k) +
 * OutT(OutT(sigmoid(g)) * s). y (tokens, k, d), w (tokens, k) float32, g (tokens), s (tokens, d). */
int sh_moe_combine(const void* y, const float* w, const void* g, const void* s, int dtype, int64_t tokens,
                   int64_t k, int64_t d, void* out, void* stream);

/* strata_mlx/blocks.py:539-563 (tiles_of): pairs of idx (pairs = tokens * k) in tiles of 16 slots of one expert.
 * tile_expert (sh_tiles_most), token (16 * most), where (pairs); workspace sh_tiles_workspace(experts) bytes. */
size_t sh_tiles_workspace(int64_t experts);
int64_t sh_tiles_most(int64_t pairs, int64_t experts);
int sh_tiles_of(const int32_t* idx, int64_t pairs, int64_t k, int64_t experts, int32_t* tile_expert, int32_t* token,
                int32_t* where, void* workspace, size_t workspace_bytes, void* stream);

/* One MoE block's decode step for tokens <= 16 (strata_mlx/fused.py:484-497, `_Routed.__call__`): top-k of the
 * router logits (float32 or the activation dtype; ties to the lower index) and the softmax of the chosen ones
 * (fused.py:491); gate/up/down of each token's experts read straight from the GGUF stacks, SwiGLU with the
 * reference's roundings (strata_mlx/blocks.py:819-829); the shared expert and its gate x . shared_gate_w; the
 * combine (fused.py:448-481). No host synchronisation: for 512 experts, d_model 2048, d_ff 512 (16-byte aligned
 * operands) two kernels (route + gate/up + SwiGLU, then down + combine), otherwise three (route; gate/up; down +
 * combine). kind / kind_down: Q2_0 or IQ3_S; dtype: F16 or BF16;
 * d_model and d_ff whole blocks of the kinds that read them (64 weights a Q2_0 block, 256 an IQ3_S one: the reference
 * model's 2560 / 640 with Q2_0 down); experts a multiple of 64 up to 2048. idx_out (tokens x k int32) and w_out
 * (tokens x k float32) are optional copies of the choice. workspace: sh_moe_workspace() bytes, zeroed once before
 * its first call (the launch's counters, at its head whatever the shape, must start at zero; every call leaves them
 * at zero, so one workspace serves calls of any shape in turn); calls sharing a workspace must not overlap. */
size_t sh_moe_workspace(int64_t tokens, int64_t k, int64_t d_model, int64_t d_ff, int dtype);
int sh_moe_decode(int kind, int kind_down, const void* gate, const void* up, const void* down, int64_t experts,
                  const void* shared_gate, const void* shared_up, const void* shared_down, const void* shared_gate_w,
                  const void* tables, const void* logits, int logits_dtype, const void* x, int dtype, int64_t tokens,
                  int64_t k, int64_t d_model, int64_t d_ff, void* out, int32_t* idx_out, float* w_out,
                  void* workspace, size_t workspace_bytes, void* stream);
/* No counterpart in the reference: sh_moe_decode for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The same arguments without the workspace: the library's
 * own device array of sh_moe_scratch_bytes() (8 MiB) on each GPU serves as it, found once per device at the first
 * call there (that first call also clears the array's counters on `stream`). Nothing is allocated. Shapes whose
 * workspace (sh_moe_workspace) exceeds the array are refused with
 * SH_E_WORKSPACE before anything is launched. Every call on a GPU shares that GPU's array: calls that overlap on one
 * GPU (two streams, two threads) race and must be ordered by the caller. */
size_t sh_moe_scratch_bytes(void);
int sh_moe_decode_noalloc(int kind, int kind_down, const void* gate, const void* up, const void* down,
                          int64_t experts, const void* shared_gate, const void* shared_up, const void* shared_down,
                          const void* shared_gate_w, const void* tables, const void* logits, int logits_dtype,
                          const void* x, int dtype, int64_t tokens, int64_t k, int64_t d_model, int64_t d_ff,
                          void* out, int32_t* idx_out, float* w_out, void* stream);
/* No counterpart in the reference (a tuning knob for callers and tests): windows of at most `upto` tokens (0..16)
 * have the routed outputs combined by the down kernel's last block of each row tile, larger ones by a combine kernel
 * after it (default 4). Both give the same bits. Returns the previous bound. Process-wide; not for use while
 * another thread launches sh_moe_decode. */
int sh_moe_set_tail_combine(int upto);
/* No counterpart in the reference: whether sh_moe_decode runs the common shape's step (512 experts, d_model 2048,
 * d_ff 512) as one launch (gate / up and down blocks in one grid) instead of two. The one-launch form is switched
 * off: on = 1 is refused with SH_E_UNSUPPORTED (it made an illegal memory access at 2 tokens; the cause is fixed,
 * the fix not yet run on a GPU); on = 0 returns the previous setting (0). */
int sh_moe_set_one_launch(int on);
/* One of sh_moe_decode's kernels alone (phase 0 route, 1 gate/up, 2 down + combine; for the two-kernel shape
 * phases 0 and 1 are both the route + gate/up kernel), in that order over one workspace: what a caller times or
 * interleaves kernel by kernel. */
int sh_moe_decode_phase(int phase, int kind, int kind_down, const void* gate, const void* up, const void* down,
                        int64_t experts, const void* shared_gate, const void* shared_up, const void* shared_down,
                        const void* shared_gate_w, const void* tables, const void* logits, int logits_dtype,
                        const void* x, int dtype, int64_t tokens, int64_t k, int64_t d_model, int64_t d_ff, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ---- prompts: the grouped expert GEMM over tiles of 16 pairs (strata_mlx/blocks.py:465-536, tile_matmul):
 * out[p] = W[tile_expert[p / 16]] . a[p] for a stack of `experts` (rows, cols) layers of `kind` blocks; a (pairs,
 * cols) bf16 or fp16 (the weights rounded to it), out (pairs, rows) fp32; rows % 64 == 0, cols % 64 == 0, pairs %
 * 16 == 0; rows of tiles naming no expert (tile_expert outside 0..experts-1) are left as they were. */
int sh_tile_matmul(int kind, const void* blocks, const void* tables, int64_t experts, int64_t rows, int64_t cols,
                   const void* a, int a_dtype, int64_t pairs, const int32_t* tile_expert, float* out, void* stream);

/* strata_mlx/blocks.py:566-574 (_tiled_glu: a = x[token]; h = swiglu(tile_matmul(gate, a), tile_matmul(up, a))
 * .astype(x.dtype)) in one pass: h[s] = x_dtype(silu(g) * u), g / u = gate / up of tile_expert[s / 16] . x[token[s]]
 * with the weights rounded to x's type and float32 sums. gate and up: stacks of `experts` (rows, cols) layers of
 * Q2_0 or IQ3_S; x (tokens, cols) bfloat16 / float16; token, h: `slots` (a multiple of 16) entries / rows; rows
 * % 32 == 0, cols % 64 == 0. Tokens outside 0..tokens-1 are clamped; tiles naming no expert leave their rows. */
int sh_tile_glu(int kind, const void* gate, const void* up, const void* tables, int64_t experts, int64_t rows,
                int64_t cols, const void* x, int x_dtype, int64_t tokens, const int32_t* token, int64_t slots,
                const int32_t* tile_expert, void* h, void* stream);

/* strata_mlx/blocks.py:575 (out = tile_matmul(down, h)[where].astype(x.dtype)) in one pass: for each slot s with
 * pair[s] in 0..pairs-1, out[pair[s]] = h_dtype(down of tile_expert[s / 16] . h[s]) (pair = the inverse of
 * tiles_of's `where`, -1 for slots no pair fills). down: Q2_0 or IQ3_S, rows % 64 == 0, cols % 64 == 0. */
int sh_tile_down(int kind, const void* down, const void* tables, int64_t experts, int64_t rows, int64_t cols,
                 const void* h, int h_dtype, int64_t slots, const int32_t* tile_expert, const int32_t* pair,
                 int64_t pairs, void* out, void* stream);
/* No counterpart in the reference (a tuning knob for callers and tests): whether the streamed tile products
 * (sh_tile_matmul, sh_tile_glu, sh_tile_down of Q2_0 / IQ3_S) share the tiles of an expert's run of at most four
 * tiles among several multiplying waves (on by default) or give each tile one wave. Both give the same bits. Read
 * at launch (a captured graph keeps the form it was captured with). Returns the previous setting. Process-wide;
 * not for use while another thread launches them. */
int sh_tiles_set_share(int on);

/* ---- dense layers: Q6_K held as three parts (strata_mlx/dense.py:109-167, ScaledLinear), w[r][c] = code[r][c] *
 * scale[r][c / 16] * d[r][c / d_step]: codes int8 (rows, cols), scales int8 (rows, cols / 16), d float16 (rows,
 * cols / d_step); rows % 4 == 0, cols % 256 == 0, d_step a multiple of 16 dividing cols. */

/* dense.py:149-167 (ScaledLinear.__call__ for a window): out[t] = W . x[t] for tokens <= 8, x and out in x_dtype
 * (F32, F16 or BF16), float32 sums. */
int sh_scaled_matvec(const int8_t* codes, const int8_t* scales, const uint16_t* d, int64_t rows, int64_t cols,
                     int64_t d_step, const void* x, int x_dtype, int64_t tokens, void* out, void* stream);
/* dense.py:120-135 (ScaledLinear.floats, kernel _FLOATS 72-82): every weight worked out in float32 and rounded
 * once to out_dtype, (rows, cols). */
int sh_scaled_floats(const int8_t* codes, const int8_t* scales, const uint16_t* d, int64_t rows, int64_t cols,
                     int64_t d_step, void* out, int out_dtype, void* stream);

/* ---- decode attention (strata_mlx/attention.py:118-165) */

/* _gathered over a page table (attention.py:144-165 with cells = page_table[p / 16] * 16 + p % 16): q (n_q, hq,
 * head_dim), k_pages / v_pages (n_pages, hkv, 16, head_dim), page_table int32 (ceil(ctx_len / 16)) of physical
 * pages; the n_q queries are the last positions of the context and query t sees positions <= ctx_len - n_q + t
 * (the causal mask among a window's drafts, attention.py:118-129). out (n_q, hq, head_dim) in `dtype` (bf16 or
 * fp16, the dtype of q, k and v); scores and sums in fp32. head_dim 128 or 256. workspace:
 * sh_paged_attn_workspace() bytes (the splits of the context). */
size_t sh_paged_attn_workspace(int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim, int64_t ctx_len);
int sh_paged_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table, int64_t n_pages,
                  int64_t ctx_len, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim, float scale, int dtype,
                  void* out, void* workspace, size_t workspace_bytes, void* stream);

/* attention.py:261 (`o_proj(out * sigmoid(gate))`): sh_paged_attn with the output gate applied in the merge,
 * out = T(T(out) * T(sigmoid(gate))); gate element (query t, head h, dim d) at gate[t * gate_token_stride + h *
 * gate_head_stride + d], in `dtype` (the second half of each head of the q projection: stride 2 head_dim a head). */
int sh_paged_attn_gated(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                        int64_t n_pages, int64_t ctx_len, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim,
                        float scale, int dtype, const void* gate, int64_t gate_token_stride, int64_t gate_head_stride,
                        void* out, void* workspace, size_t workspace_bytes, void* stream);

/* attention.py:183-222 (`qk_rope`, kernel _QK_ROPE 183-214): q or k of a window, x (tokens, heads, stride) with each
 * head's head_dim values first: each head's rms norm with `weight` (head_dim) and eps, then rope on the first `rot`
 * dims with cos / sin (tokens, rot), every step rounded to `dtype` as the reference's kernel does. out (heads,
 * tokens, head_dim) when heads_first, else (tokens, heads, head_dim). head_dim a multiple of 64 up to 512. */
int sh_qk_rope(const void* x, int dtype, int64_t tokens, int64_t heads, int64_t head_dim, int64_t stride,
               const void* weight, float eps, const void* cos, const void* sin, int64_t rot, void* out, int heads_first,
               void* stream);

/* attention.py:251 (`cache.update_and_fetch(k, v)` of a paged cache): the window's keys and values k, v (n_new,
 * hkv, head_dim) written at positions pos0 .. pos0 + n_new - 1, position p to page page_table[p / 16], slot p % 16
 * of the pools (n_pages, hkv, 16, head_dim). page_table holds table_pages entries: positions past 16 table_pages
 * are refused with SH_E_SHAPE. Page ids outside 0..n_pages-1 are not written. Trimming rejected
 * drafts is the caller's position count alone (the pages keep what they hold until written again). */
int sh_kv_append(const void* k, const void* v, int64_t n_new, int64_t hkv, int64_t head_dim, int dtype, void* k_pages,
                 void* v_pages, const int32_t* page_table, int64_t table_pages, int64_t n_pages, int64_t pos0,
                 void* stream);

/* _gathered in its own form (attention.py:132-165): query s attends to the n_cells cells cells[s] (int32, rows of
 * k / v (hkv, kv_len, head_dim)) whose flag real[s] (uint8) is set; q (n_q, hq, head_dim) -> out (n_q, hq,
 * head_dim). workspace: sh_cells_attn_workspace() bytes. */
size_t sh_cells_attn_workspace(int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim, int64_t n_cells);
int sh_cells_attn(const void* q, const void* k, const void* v, int64_t kv_len, const int32_t* cells,
                  const uint8_t* real, int64_t n_cells, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim,
                  float scale, int dtype, void* out, void* workspace, size_t workspace_bytes, void* stream);

/* attention.py:144-165 (`_gathered`) over a paged pool: the cells of sh_cells_attn (positions 0 .. n_pages * 16 - 1)
 * read from pages (n_pages, hkv, 16, head_dim), position p at page page_table[p / 16], slot p % 16; `gate` (nullable)
 * as in sh_paged_attn_gated. The attention entry's path for queries with an indexer's choice (attention.py:255-256). */
int sh_cells_attn_paged(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                        int64_t n_pages, const int32_t* cells, const uint8_t* real, int64_t n_cells, int64_t n_q,
                        int64_t hq, int64_t hkv, int64_t head_dim, float scale, int dtype, const void* gate,
                        int64_t gate_token_stride, int64_t gate_head_stride, void* out, void* workspace,
                        size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRATA_HIP_H */

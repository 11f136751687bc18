/*
 * libccq_hip -- C ABI of the MI355X (gfx950) quantized expert-matmul path.
 *
 * The reference (CostCut-Infer) has no FFI: its boundary is a set of Python
 * callables.  Each entry point below names the reference callable it replaces
 * (file:line under python/ccut/).  Python binds this header with ctypes
 * (costcut-infer_amd/ccut/_lib.py).
 *
 * Rules common to every entry point:
 *   - return 0 on success; CCQ_EINVAL / CCQ_EUNSUPPORTED / CCQ_EWORKSPACE
 *     (< 0) for argument errors, detected on the host before any launch (the
 *     message is in ccq_last_error(), thread-local); > 0 is a hipError_t
 *     reported by the launch;
 *   - every pointer is a caller-allocated DEVICE pointer unless stated;
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); work is
 *     stream-ordered and asynchronous; nothing here allocates memory;
 *   - matrices are row-major and dense (leading dimension = row length).
 */
#ifndef CCQ_H_
#define CCQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CCQ_EINVAL (-1)
#define CCQ_EUNSUPPORTED (-2)
#define CCQ_EWORKSPACE (-3)

/* element types of activations / outputs / scales */
#define CCQ_F32 0
#define CCQ_F16 1
#define CCQ_BF16 2

/* library version (major*10000 + minor*100 + patch) */
int ccq_version(void);
/* message of the last failed call on this thread ("" if none) */
const char* ccq_last_error(void);

/* Kernel-exact timing, for benchmarks: the next kernel that a ccq entry
 * point launches on this thread records start_event when it begins
 * executing and stop_event when it ends (hipExtLaunchKernel), so
 * hipEventElapsedTime(start, stop) is that kernel's own duration -- the
 * interval rocprofv3's kernel trace reports -- without the gap between
 * back-to-back launches.  Applies to one launch, then clears; both events
 * (hipEvent_t, created with timing) or neither (clears).  No counterpart in
 * the reference: its kernels are host code. */
int ccq_launch_timer(void* start_event, void* stop_event);

/* ------------------------------------------------------------------------
 * Reference formats (exact reference semantics, float32 I/O)
 * ---------------------------------------------------------------------- */

/* e4m3fn bytes -> float32, n elements.
 * Replaces fp8_e4m3_to_float32 (quant/kernels.py:52-74). */
int ccq_fp8_to_f32(const uint8_t* code, float* out, int64_t n, void* stream);

/* float32 -> e4m3fn with the reference's round-half-up, saturation to 448
 * (>= 464), NaN -> 0x7F, -0.0 -> 0x00.
 * Replaces float32_to_fp8_e4m3 (quant/kernels.py:77-123). */
int ccq_f32_to_fp8(const float* x, uint8_t* out, int64_t n, void* stream);

/* Load-time FP8 quantization of a BF16 weight [rows, cols] (row-major
 * bf16 bits) to e4m3 codes [rows, cols], per output row: scale[r] when
 * scale is non-null, else amax(|row|)/448 (0 -> 1); scales <= 0 or NaN
 * -> 1; code = the reference's half-up encoding of clip(w / s, +-448)
 * (float32 division).  Replaces quantize_buffer_inplace
 * (quant/online.py:37-64). */
int ccq_quantize_rows_fp8(const uint16_t* w_bf16, const float* scale, uint8_t* out, int64_t rows,
                          int64_t cols, void* stream);

/* Per-token KV cache quantization: kv [rows, dim] f32 (rows = 2 * heads *
 * seq) -> codes [rows, dim] e4m3 and one e4m3 scale byte per row:
 * amax <= 0 -> zeros; else s = amax/448, codes = half-up(clip(x / s)),
 * scale = half-up(s).  Replaces quantize_kv_token (quant/kv.py:70-90). */
int ccq_kv_quant_fp8(const float* kv, uint8_t* out, uint8_t* scales, int64_t rows, int64_t dim, void* stream);

/* KV read-back: out = fp8(code) * fp8(scale) (float32) where the scale
 * decodes to > 0, else 0.  Replaces dequantize_kv_token (quant/kv.py:93-101). */
int ccq_kv_dequant_fp8(const uint8_t* codes, const uint8_t* scales, float* out, int64_t rows, int64_t dim,
                       void* stream);

/* out[r,c] = fp8(w[r,c]) * scale[r]   (w [rows,cols] e4m3fn, scale [rows]).
 * Replaces fp8_dequant_mat / fp8_dequant_row (quant/kernels.py:126-171). */
int ccq_fp8_dequant(const uint8_t* w, const float* scale, float* out,
                    int64_t rows, int64_t cols, void* stream);

/* out[i * group_size + j] = scale_groups[i] for i < groups, j < group_size
 * (float32; out holds at least groups * group_size elements, the rest is
 * left as it is).  Replaces group_broadcast_scale (quant/kernels.py:258-268). */
int ccq_group_broadcast_scale(const float* scale_groups, int64_t groups, int64_t group_size, float* out,
                              void* stream);

/* out = gate / (1 + exp(-gate)) * up, computed in float64, stored float32.
 * Replaces silu_mul_fused (quant/kernels.py:219-231). */
int ccq_silu_mul(const float* gate, const float* up, float* out, int64_t n, void* stream);

/* Reference int4: signed nibbles, low nibble first, one scale per INPUT column.
 * packed [rows, cols/2] u8, scale [cols] f32 -> out [rows, cols] f32.
 * Replaces int4_dequant_row (quant/kernels.py:276-295). */
int ccq_int4_dequant(const uint8_t* packed, const float* scale, float* out,
                     int64_t rows, int64_t cols, void* stream);

/* y[b, r] = sum_c x[b,c] * W[r,c] in float32, W dequantized on the fly exactly
 * as ccq_int4_dequant.  x [batch, in] f32, packed [out, in/2], y [batch, out].
 * Replaces WeightOnlyMethod.apply (quant/weight_only.py:37-54). */
int ccq_int4_linear_f32(const float* x, const uint8_t* packed, const float* scale,
                        float* y, int64_t batch, int64_t in_features,
                        int64_t out_features, void* stream);

/* NF4: packed as ccq_int4_dequant (low nibble = even column, scale per input
 * column), W[r,c] = table[code] * scale[c] for code < table_len, NaN past
 * the table (the reference's 8-entry table is indexed by the 4-bit code
 * unchecked).  table: table_len (<= 16) float32 on the device.  Replace
 * kernels.nf4_dequant_row (quant/kernels.py:299-322) and WeightOnlyMethod.apply
 * for NF4 (quant/weight_only.py:37-54). */
int ccq_nf4_dequant(const uint8_t* packed, const float* scale, const float* table,
                    int table_len, float* out, int64_t rows, int64_t cols, void* stream);
int ccq_nf4_linear_f32(const float* x, const uint8_t* packed, const float* scale,
                       const float* table, int table_len, float* y, int64_t batch,
                       int64_t in_features, int64_t out_features, void* stream);

/* Per-column int8 quantization of x [rows, cols] with a given amax [cols]:
 * inv = 127 / amax (float64; 0 when amax is not > 0), q = round-half-even(
 * x * inv) clamped to +-127 (NaN -> 0, +-inf -> +-127: undefined in the
 * reference).  Replaces kernels.int8_quantize_row (quant/kernels.py:192-211). */
int ccq_int8_quantize_cols(const float* x, const float* amax, int8_t* out,
                           int64_t rows, int64_t cols, void* stream);

/* y[b, r] = sum_c x[b,c] * fp8(w[r,c]) * scale[r] in float32.
 * Replaces LinearMethod.apply w8a16 / w8a8 (quant/method.py:100-140) and
 * Fp8LinearMethod.apply (quant/fp8.py:33). */
int ccq_fp8_linear_f32(const float* x, const uint8_t* w, const float* scale,
                       float* y, int64_t batch, int64_t in_features,
                       int64_t out_features, void* stream);

/* y[b, r] = sum_c x[b,c] * (w[r,c] * scale[r]) in float32, w int8 [out, in],
 * one scale per output row (the W8A16 path).  Replaces Int8LinearMethod.apply
 * with compute_path "w8a16" (quant/int8.py:38-50) and LinearMethod.apply for
 * int8 keys (quant/method.py:106-111,126-130). */
int ccq_int8_linear_f32(const float* x, const int8_t* w, const float* scale,
                        float* y, int64_t batch, int64_t in_features,
                        int64_t out_features, void* stream);

/* Bytes of workspace ccq_int8_w8a8_linear needs for this shape (0: none). */
size_t ccq_int8_w8a8_workspace_size(int64_t M, int64_t K, int64_t N);

/* The whole W8A8 layer from float32 activations: x_scale[M] and y[M, N] as
 * ccq_int8_act_quant followed by ccq_int8_linear give them, bit for bit.
 * Up to 4 rows the activation quantization runs inside the GEMM (one
 * launch); otherwise the quantized rows go to the workspace.  K > 0.
 * Replaces Int8LinearMethod._w8a8 (quant/int8.py:52-62). */
int ccq_int8_w8a8_linear(const float* x, float* x_scale, const int8_t* w,
                         const float* w_scale, float* y, int64_t M, int64_t K,
                         int64_t N, void* workspace, size_t workspace_bytes,
                         void* stream);

/* out[r, c] = w[r, c] * scale[r] (float32).  Replaces kernels.int8_dequant_row
 * (quant/kernels.py:180-189). */
int ccq_int8_dequant(const int8_t* w, const float* scale, float* out,
                     int64_t rows, int64_t cols, void* stream);

/* Per-token symmetric int8 activation quantization: amax = max|x[m,:]| (NaN
 * if the row holds one), amax' = amax > 0 ? amax : 1, x_scale[m] = amax'/127,
 * factor = 127/x_scale[m] (float32 divisions), xq = clamp(rint(x*factor),
 * -127, 127), NaN -> 0.  x [M, K] f32.  Replaces _quantize_per_token
 * (quant/int8.py:65-77). */
int ccq_int8_act_quant(const float* x, int8_t* xq, float* x_scale,
                       int64_t M, int64_t K, void* stream);

/* E8M0 scale bytes -> float32: 2^(e-127), e = 0 -> 0, e = 255 -> NaN.
 * Replaces kernels.mx_e8m0_to_float (quant/kernels.py:240-256). */
int ccq_e8m0_to_f32(const uint8_t* e8m0, float* out, int64_t n, void* stream);

/* MX weights [rows, cols] -> float32, groups of group_size columns per row
 * with E8M0 scales [rows, ceil(cols / group_size)].  fmt 0 MXFP8 (e4m3fn
 * bytes, scales required): W = fp8(w) * s.  fmt 1 MXFP4 / NVFP4 (two codes
 * per byte, low nibble first; scales may be NULL): W = (lut[code] * s) *
 * scale2, lut = {0, .5, 1, 1.5, -0, -.5, -1, -1.5} for codes & 7.  Replaces
 * MxLinearMethod._dequant_mx / _dequant_mx4 (quant/mx.py:60-94, the NVFP4
 * factor of :55-56). */
int ccq_mx_dequant(const uint8_t* w, const uint8_t* scale_e8m0, float* out,
                   int64_t rows, int64_t cols, int fmt, int group_size,
                   float scale2, void* stream);

/* y[b, r] = sum_c x[b,c] * W[r,c] in float32, W as ccq_mx_dequant forms it.
 * Replaces MxLinearMethod.apply (quant/mx.py:37-58). */
int ccq_mx_linear_f32(const float* x, const uint8_t* w, const uint8_t* scale_e8m0,
                      float* y, int64_t batch, int64_t in_features,
                      int64_t out_features, int fmt, int group_size,
                      float scale2, void* stream);

/* y[b, r] = sum_c x[b,c] * W[r,c] in float32 on the matrix cores: each
 * weight decoded in registers to its exact bf16 value, x split into bf16
 * hi + lo (float32-grade products), W read once per 64 batch rows.
 * fmt 0: e4m3fn codes [out, in] with a float32 scale per row (scale float*);
 * 1: int8 codes, float32 row scale; 2: MXFP8 (E8M0 scales [out, in/G],
 * G 16 or 32); 3: MXFP4 / NVFP4 codes as ccq_mx_dequant (scales optional,
 * scale2 on each sum).  in_features a positive multiple of 256; x and w
 * 16-byte aligned.  The batched form of Fp8LinearMethod.apply
 * (quant/fp8.py:35-42), LinearMethod.apply for fp8 / int8 keys
 * (quant/method.py:100-140) and MxLinearMethod.apply (quant/mx.py:37-58):
 * ccq_mx_linear_f32 calls it for every batch, ccq_fp8_linear_f32 from 2
 * rows and ccq_int8_linear_f32 from 4 rows on (where it measured faster). */
int ccq_wq_mfma_linear_f32(const float* x, const uint8_t* w, const void* scale,
                           float* y, int64_t batch, int64_t in_features,
                           int64_t out_features, int fmt, int group_size,
                           float scale2, void* stream);

/* Bytes of workspace ccq_int8_linear needs for this shape (0: none). */
size_t ccq_int8_linear_workspace_size(int64_t M, int64_t K, int64_t N);

/* W8A8: acc[m,n] = sum_k xq[m,k] * w[n,k] exactly (int32; K < 131072),
 * y[m,n] = (float(acc) * x_scale[m]) * w_scale[n] in float32.  xq [M, K],
 * w [N, K] int8.  Replaces Int8LinearMethod._w8a8 after the activation
 * quantization and _int8_matmul (quant/int8.py:52-62,80-100). */
int ccq_int8_linear(const int8_t* xq, const float* x_scale, const int8_t* w,
                    const float* w_scale, float* y, int64_t M, int64_t K,
                    int64_t N, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ------------------------------------------------------------------------
 * AWQ int4 (qweight int32 [K, N/8] AWQ order, qzeros int32 [K/G, N/8],
 * scales f16|bf16 [K/G, N]; W[k,n] = (q - z) * s; y = x @ W)
 * The reference only names these tensors (quant/compressed_tensors.py:209-211)
 * and has no arithmetic for them; these entry points sit behind the same
 * QuantizeMethodBase.apply boundary (quant/method.py:45-58).
 * ---------------------------------------------------------------------- */

/* W [K, N] float32, bit-exact (q - z) * s.  scale_dtype CCQ_F16 | CCQ_BF16. */
int ccq_awq_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                    int scale_dtype, float* out, int64_t K, int64_t N,
                    int64_t group_size, void* stream);

/* Re-pack qweight [K, N/8] into the gfx950 tile layout used by every GEMM
 * below (same byte count: K*N/2).  Requires K % 128 == 0, N % 16 == 0.
 * Load-time step, the hook of QuantizeMethodBase.process_weights_after_loading
 * (quant/method.py:60-62).  `tiled` must not alias `qweight`. */
int ccq_awq_repack(const int32_t* qweight, int32_t* tiled, int64_t K, int64_t N,
                   void* stream);

/* Inverse of ccq_awq_repack (test/export helper). */
int ccq_awq_unpack_tiled(const int32_t* tiled, int32_t* qweight, int64_t K, int64_t N,
                         void* stream);

/* 32-bit words per output column of the packed scale/zero array ("SZ"):
 * K/G groups, padded to whole chunks of 4 k-tiles (0 for invalid shapes). */
int64_t ccq_awq_sz_words(int64_t K, int64_t group_size);

/* Pack qzeros [K/G, N/8] and scales [K/G, N] (scale_dtype CCQ_F16|CCQ_BF16)
 * into sz [N, ccq_awq_sz_words(K, G)] uint32: word [n][g] = scale bits |
 * zero << 16, padding words 0.  Load-time step next to ccq_awq_repack. */
int ccq_awq_pack_sz(const int32_t* qzeros, const void* scales, int scale_dtype,
                    uint32_t* sz, int64_t K, int64_t N, int64_t group_size, void* stream);

/* Workspace bytes ccq_w4_gemm needs for these sizes: 0 for the decode
 * kernels (M <= 64, or group_size != 128, or N % 128 != 0, or K < 256),
 * else the per-row group sums of x (M * K/128 floats) and the row ids of
 * the 128-row tiles, each 256-byte rounded. */
size_t ccq_w4_gemm_workspace_size(int64_t M, int64_t K, int64_t N, int64_t group_size);

/* y [M, N] = x [M, K] @ dequant(W) with fp32 accumulation.
 * x_dtype CCQ_F16 | CCQ_BF16; scale_dtype (of the scales packed in sz)
 * CCQ_F16 | CCQ_BF16; y_dtype CCQ_F16 | CCQ_BF16 | CCQ_F32.  w_tiled from
 * ccq_awq_repack, sz from ccq_awq_pack_sz.  group_size in {32, 64, 128}.
 * x, w_tiled and sz must be 16-byte aligned.  M <= 16 with group 128 and
 * K <= 4096: the persistent streaming kernel (weights read once); other
 * M <= 64: one workgroup per 16-row tile and column block (one weight pass
 * per 16 rows); no workspace for either.  Larger M with group 128,
 * N % 128 == 0 and K >= 256: the grouped MFMA kernel over 128-row tiles,
 * which needs ccq_w4_gemm_workspace_size bytes (256-byte aligned).
 * Replaces WeightOnlyMethod.apply (quant/weight_only.py:37-54) for AWQ. */
int ccq_w4_gemm(const void* x, int x_dtype, const int32_t* w_tiled,
                const uint32_t* sz, int scale_dtype,
                void* y, int y_dtype, int64_t M, int64_t K, int64_t N,
                int64_t group_size, void* workspace, size_t workspace_bytes,
                void* stream);

/* ------------------------------------------------------------------------
 * Routing and token grouping
 * ---------------------------------------------------------------------- */

/* Top-k routing weights.  logits [T, E] f32 -> weights [T, k] f32,
 * ids [T, k] int64.  mode 1: top-k of the logits then softmax over the k
 * (topk_softmax norm_topk_prob=True, blocks/moe.py:84-89); mode 0: softmax
 * over all E then top-k of the probabilities (norm_topk_prob=False,
 * blocks/moe.py:79-83); mode 2: exp(v)/sum(exp(v)) over the k raw logits
 * (route_experts norm_topk=0, blocks/moe.py:113-118); mode 3: plain top-k,
 * weights = the selected logits (topk, blocks/moe.py:46-68); mode 4:
 * exp(v - max)/sum over the k (route_experts norm_topk=1,
 * blocks/moe.py:100-112).  Modes 0 and 1 divide by numpy's
 * maximum(sum, 1e-30), which keeps a NaN sum (a NaN or +inf logit makes the
 * row NaN); modes 2 and 4 sum in float64 and give 0 when the sum is not
 * > 0.  Selection is topk (blocks/moe.py:46-68): strict '>', ties to the
 * lowest index.
 * E <= 1024, 1 <= k <= 16, k <= E. */
int ccq_topk_softmax(const float* logits, float* weights, int64_t* ids,
                     int64_t T, int64_t E, int64_t k, int mode, void* stream);

/* Upper bound of the number of tiles ccq_moe_align can emit. */
int64_t ccq_moe_align_max_tiles(int64_t num_assignments, int64_t num_experts, int64_t tile_m);

/* Expert-sorted, tile-padded schedule of the T*k assignments (a = t*k+slot).
 * Experts in first-appearance order (t ascending, then slot), assignments
 * ascending within an expert: the permutation of moe_combine
 * (blocks/moe.py:163-167) and moe_forward (models/generic.py:366-370).
 * Outputs: sorted_ids [max_tiles*tile_m] int32 (-1 = padding),
 * tile_expert [max_tiles] int32, meta[0] = number of tiles,
 * meta[1] = number of distinct experts, counts [E] int32 per expert.
 * ids outside [0, E) are dropped.  num_assignments <= 65536, E <= 1024. */
int ccq_moe_align(const int64_t* ids, int64_t num_assignments, int64_t num_experts,
                  int64_t tile_m, int32_t* sorted_ids, int32_t* tile_expert,
                  int32_t* meta, int32_t* counts, void* stream);

/* y[t, :] = sum_{s<k} weights[t,s] * rows[t*k+s, :]   (slot order, fp32 sum).
 * rows [T*k, H] f32; y dtype CCQ_F32 | CCQ_BF16 | CCQ_F16.
 * The weighted combine of moe_combine (blocks/moe.py:172-173). */
int ccq_moe_combine(const float* rows, const float* weights, void* y, int y_dtype,
                    int64_t T, int64_t k, int64_t H, void* stream);

/* ccq_moe_combine with the shared expert's add in its epilogue:
 * y[t, :] = sum (as above) + float32(shared_gate * shared[t, :]), shared
 * [T, H] f32.  The combine of moe_combine followed by shared_expert_add
 * (blocks/moe.py:172-179; experts/pipeline.py:181-190). */
int ccq_moe_combine_shared(const float* rows, const float* weights, const float* shared,
                           float shared_gate, void* y, int y_dtype, int64_t T, int64_t k,
                           int64_t H, void* stream);

/* y[i] += float32(shared_gate * shared[i]) in place, float32 (the product
 * rounded, then the add).  Replaces shared_expert_add (blocks/moe.py:177-179). */
int ccq_shared_expert_add(float* y, const float* shared, float shared_gate, int64_t n,
                          void* stream);

/* ------------------------------------------------------------------------
 * MoE expert FFN, AWQ int4 experts (gate/up [H -> I], down [I -> H])
 * Weights of all E experts are stacked: w_gate/w_up tiled [E][H*I/8] int32
 * (ccq_awq_repack), sz_gate/sz_up [E][I][ccq_awq_sz_words(H, G)];
 * w_down [E][I*H/8], sz_down [E][H][ccq_awq_sz_words(I, G)]
 * (ccq_awq_pack_sz).
 * Replaces expert_ffn (blocks/moe.py:122-141) + moe_combine
 * (blocks/moe.py:144-174) as called by ExpertPipeline.step
 * (experts/pipeline.py:155-179) and moe_forward (models/generic.py:348-378).
 * ---------------------------------------------------------------------- */

typedef struct ccq_w4_experts {
  const int32_t* w_gate; const uint32_t* sz_gate;
  const int32_t* w_up;   const uint32_t* sz_up;
  const int32_t* w_down; const uint32_t* sz_down;
  int scale_dtype;           /* CCQ_F16 | CCQ_BF16 (scales inside sz) */
  int64_t num_experts, hidden, inter, group_size;
} ccq_w4_experts;

/* Stage entry points of ccq_moe_w4_ffn, for callers that build the schedule
 * themselves with ccq_moe_align (tile_m = 16, max_tiles from
 * ccq_moe_align_max_tiles).  Rows are assignments a = t*k + slot.
 * gate_up: inter[a, :] = silu(x[a/k] @ Wg_e) * (x[a/k] @ Wu_e), x_dtype out.
 * down:    rows[a, :]  = inter[a] @ Wd_e, float32.
 * Stage calls need no workspace. */
int ccq_moe_w4_gate_up(const void* x, int x_dtype, int64_t k, const int32_t* sorted_ids,
                       const int32_t* tile_expert, const int32_t* meta, int64_t max_tiles,
                       void* inter, const ccq_w4_experts* ex, void* stream);
int ccq_moe_w4_down(const void* inter, int x_dtype, const int32_t* sorted_ids,
                    const int32_t* tile_expert, const int32_t* meta, int64_t max_tiles,
                    float* rows, const ccq_w4_experts* ex, void* stream);

/* Workspace bytes for ccq_moe_w4_ffn (schedule, intermediate and down rows;
 * no initial contents required).  Calls sharing one workspace must not
 * overlap in time. */
size_t ccq_moe_w4_workspace_size(int64_t T, int64_t k, const ccq_w4_experts* ex);

/* Full MoE FFN from routing: x [T, H] (x_dtype CCQ_BF16 | CCQ_F16),
 * ids [T, k] int64 and weights [T, k] f32 (from ccq_topk_softmax),
 * y [T, H] (y_dtype CCQ_BF16 | CCQ_F16 | CCQ_F32). */
int ccq_moe_w4_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights,
                   void* y, int y_dtype, int64_t T, int64_t k,
                   const ccq_w4_experts* ex, void* workspace, size_t workspace_bytes,
                   void* stream);

/* ccq_moe_w4_ffn with the shared expert's output shared [T, H] f32 added in
 * the combine's epilogue as ccq_moe_combine_shared does (the routed FFN,
 * combine and shared_expert_add of ExpertPipeline.step,
 * experts/pipeline.py:145-190, in one call). */
int ccq_moe_w4_ffn_shared(const void* x, int x_dtype, const int64_t* ids, const float* weights,
                          const float* shared, float shared_gate, void* y, int y_dtype,
                          int64_t T, int64_t k, const ccq_w4_experts* ex, void* workspace,
                          size_t workspace_bytes, void* stream);

/* The MoE layer from router logits: routing (ccq_topk_softmax, mode as
 * there) + ccq_moe_w4_ffn in one call.  logits [T, E] f32 with
 * E = ex->num_experts; ids_out [T, k] int64 and weights_out [T, k] f32
 * receive the routing (either may be null: the workspace keeps it);
 * workspace as ccq_moe_w4_ffn.  Decode batches (T <= 16, T*k <= 256, E <= 256,
 * T*E <= 4096, k <= 16) route inside the gate/up kernel's workgroups (three launches in
 * all; two when T*k <= 16, whose down kernel also combines); larger ones run
 * the routing kernel and ccq_moe_w4_ffn.  Same results either way.  Replaces moe_forward (models/generic.py:348-378): topk_softmax
 * + expert grouping + expert_ffn + combine. */
int ccq_moe_w4_forward(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k,
                       int mode, int64_t* ids_out, float* weights_out, void* y, int y_dtype,
                       const ccq_w4_experts* ex, void* workspace, size_t workspace_bytes,
                       void* stream);

/* The first of ccq_moe_w4_forward's launches for a decode batch: the
 * gate/up + SiLU kernel that routes the batch inside its workgroups, leaving
 * the routing (ids_out / weights_out, or the workspace), the expert schedule
 * and the intermediate in the workspace exactly as ccq_moe_w4_forward does
 * before its down and combine launches.  Arguments as ccq_moe_w4_forward
 * (no output); CCQ_EUNSUPPORTED for batches that ccq_moe_w4_forward routes
 * with the separate routing kernel.  The stage the forward's routing and
 * gate/up share with ccq_moe_w4_gate_up (experts/pipeline.py:145-170). */
int ccq_moe_w4_route_gate_up(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k,
                             int mode, int64_t* ids_out, float* weights_out, const ccq_w4_experts* ex,
                             void* workspace, size_t workspace_bytes, void* stream);

/* The MoE layer with its shared expert's FFN in the same kernels: ex holds
 * E = num_experts - 1 routed experts and the shared expert last (index E);
 * logits are [T, E].  Every token takes the shared expert as one more
 * assignment slot (slot k, weight shared_gate), so its gate/up + SiLU and
 * down run inside the routed experts' launches and the combine adds
 * shared_gate * shared(x) after the routed sum, in the reference's order:
 * y = sum_j w_j * expert_ffn(x, e_j) + shared_gate * shared_ffn(x)
 * (experts/pipeline.py:145-190, blocks/moe.py:177-179).  k <= 15;
 * ids_out / weights_out, when given, are [T, k + 1] (the shared slot
 * last); the workspace is ccq_moe_w4_workspace_size(T, k + 1, ex). */
int ccq_moe_w4_forward_shared(const void* x, int x_dtype, const float* logits, int64_t T,
                              int64_t k, int mode, float shared_gate, int64_t* ids_out,
                              float* weights_out, void* y, int y_dtype, const ccq_w4_experts* ex,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the per-GPU scratch array of ccq_moe_w4_forward_noalloc. */
#define CCQ_MOE_W4_NOALLOC_BYTES (32u << 20)

/* ccq_moe_w4_forward with no workspace argument: same arguments otherwise,
 * same kernels, same results bit for bit.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * workspace is a static device array of CCQ_MOE_W4_NOALLOC_BYTES held by
 * every GPU the library runs on until the process ends; a call whose
 * ccq_moe_w4_workspace_size(T, k, ex) exceeds it fails with CCQ_EINVAL
 * before any launch (at 64 experts, hidden 2048, inter 1408, top-6 that is
 * T above about 500).  Nothing is allocated.  Calls that overlap in time on
 * one GPU share the array and race: serialize them (one stream, or events). */
int ccq_moe_w4_forward_noalloc(const void* x, int x_dtype, const float* logits, int64_t T, int64_t k,
                               int mode, int64_t* ids_out, float* weights_out, void* y, int y_dtype,
                               const ccq_w4_experts* ex, void* stream);


/* ------------------------------------------------------------------------
 * FP8 e4m3fn with 128x128 block weight scales (w [N, K] bytes, row = output
 * channel, s_w [N/128, K/128] f32: W[n,k] = fp8(w[n,k]) * s_w[n/128, k/128])
 * and per-token-per-128 dynamic activation scales.  The reference has FP8
 * with one scale per output row only (quant/kernels.py:150-171) and its
 * "w8a8" does not quantize activations (quant/method.py:133-140); these
 * entry points serve the block-scaled layout behind the same
 * Fp8LinearMethod.apply boundary (quant/fp8.py:33, quant/method.py:45-58).
 * ---------------------------------------------------------------------- */

/* q [rows, K] e4m3fn, s [rows, K/128] f32: s = max(amax, 1e-12) / 448 over
 * each 128-column block of a row, q = RNE(x / s) saturated to +-448.
 * x_dtype CCQ_F32 | CCQ_F16 | CCQ_BF16, K % 128 == 0, q 8-byte aligned. */
int ccq_fp8_act_quant(const void* x, int x_dtype, int64_t rows, int64_t K,
                      uint8_t* q, float* s, void* stream);

/* Re-pack w [N, K] e4m3fn into the gfx950 MFMA tile layout (same bytes):
 * 2 KiB chunks per (16-column tile, 128-wide K block), the 8 tiles of each
 * 128-column block contiguous at each K block; N % 128 == 0, K % 128 == 0,
 * 16-byte aligned, not in place.  Load-time step
 * (QuantizeMethodBase.process_weights_after_loading, quant/method.py:60-62). */
int ccq_fp8_block_repack(const uint8_t* w, uint8_t* tiled, int64_t N, int64_t K,
                         void* stream);
/* Inverse of ccq_fp8_block_repack. */
int ccq_fp8_block_unpack(const uint8_t* tiled, uint8_t* w, int64_t N, int64_t K,
                         void* stream);

/* out [N, K] f32 = fp8(w[n, k]) * s_w[n/128, k/128] (one float32
 * rounding), any N, K; s_w [ceil(N/128), ceil(K/128)].  The per-expert
 * weight-unpack stage of ExpertReader._fill / _dequant_seg
 * (experts/reader.py:142-251) for block-scaled FP8 checkpoints
 * (weight_scale_inv), whose per-row form is ccq_fp8_dequant. */
int ccq_fp8_block_dequant(const uint8_t* w, const float* s_w, float* out, int64_t N, int64_t K,
                          void* stream);

/* Workspace of ccq_fp8_block_linear (the quantized activations). */
size_t ccq_fp8_block_linear_workspace_size(int64_t M, int64_t K);

/* y [M, N] = dequant(act_quant(x)) @ W^T with fp32 accumulation;
 * K % 128 == 0 and K >= 256 (or K == 0), N % 128 == 0, w_tiled from
 * ccq_fp8_block_repack. */
int ccq_fp8_block_linear(const void* x, int x_dtype, const uint8_t* w_tiled,
                         const float* s_w, void* y, int y_dtype, int64_t M, int64_t K,
                         int64_t N, void* workspace, size_t workspace_bytes,
                         void* stream);

/* MoE experts, FP8 block: gate/up w [E][I, H] (tiled), s [E][I/128][H/128];
 * down w [E][H, I] (tiled), s [E][H/128][I/128]. */
typedef struct ccq_fp8_experts {
  const uint8_t* w_gate; const float* s_gate;
  const uint8_t* w_up;   const float* s_up;
  const uint8_t* w_down; const float* s_down;
  int64_t num_experts, hidden, inter;
} ccq_fp8_experts;

/* Workspace bytes of ccq_moe_fp8_ffn (schedule, quantized activations and
 * intermediate, down rows; no initial contents required). */
size_t ccq_moe_fp8_workspace_size(int64_t T, int64_t k, const ccq_fp8_experts* ex);

/* Full MoE FFN on FP8 block experts: x [T, H] is quantized per token per
 * 128; gate/up + SiLU*up with the intermediate rounded to bf16 and
 * re-quantized per row per 128; down; weighted combine in slot order.
 * Tokens are grouped by expert into 128-row tiles (ccq_moe_align);
 * hidden and inter must be multiples of 128 and at least 256.
 * Replaces expert_ffn + moe_combine (blocks/moe.py:122-174) for FP8
 * experts, as called by moe_forward (models/generic.py:348-378). */
int ccq_moe_fp8_ffn(const void* x, int x_dtype, const int64_t* ids, const float* weights,
                    void* y, int y_dtype, int64_t T, int64_t k,
                    const ccq_fp8_experts* ex, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ccq_moe_fp8_ffn with the shared expert's output shared [T, H] f32 added
 * in the combine's epilogue, as ccq_moe_w4_ffn_shared does. */
int ccq_moe_fp8_ffn_shared(const void* x, int x_dtype, const int64_t* ids, const float* weights,
                           const float* shared, float shared_gate, void* y, int y_dtype,
                           int64_t T, int64_t k, const ccq_fp8_experts* ex, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * MoE experts in the reference's own checkpoint format: FP8 e4m3 codes
 * [out, in] with one float32 scale per output row (the checkpoint's BF16
 * [out, 1] scale, widened), as ExpertReader._fill / _dequant_seg read them
 * (experts/reader.py:142-251): gate/up w [E][I][H], s [E][I]; down
 * w [E][H][I], s [E][H].  Used in place: no re-pack.
 * ---------------------------------------------------------------------- */
typedef struct ccq_fp8row_experts {
  const uint8_t* w_gate; const float* s_gate;
  const uint8_t* w_up;   const float* s_up;
  const uint8_t* w_down; const float* s_down;
  int64_t num_experts, hidden, inter;
} ccq_fp8row_experts;

/* Workspace bytes of ccq_moe_fp8row_ffn (schedule, float32 intermediate and
 * down rows; no initial contents required). */
size_t ccq_moe_fp8row_workspace_size(int64_t T, int64_t k, const ccq_fp8row_experts* ex);

/* The routed experts' FFN and weighted combine on per-row FP8 experts, in
 * the reference's float32 arithmetic: x [T, H] f32, ids [T, k] int64,
 * weights [T, k] f32 (ids outside [0, E) contribute nothing), y [T, H]
 * (y_dtype CCQ_F32 | CCQ_BF16 | CCQ_F16).  For each routed expert e:
 * h = silu(x W_g^T) * (x W_u^T), rows = h W_d^T with W = fp8(w) * s[row]
 * (products exact: weights decoded to bf16, activations split into bf16
 * hi + lo; float32 accumulation; SiLU product in float64, rounded once);
 * y[t] = sum over slots of weights[t,s] * rows[t,s] in slot order.
 * hidden and inter must be multiples of 256, T*k <= 65536, E <= 1024.
 * Replaces the per-expert loop of ExpertPipeline.step
 * (experts/pipeline.py:155-179): reader.get + expert_ffn
 * (blocks/moe.py:122-141) + the weighted add, for reader slots in this
 * format. */
int ccq_moe_fp8row_ffn(const float* x, const int64_t* ids, const float* weights, void* y, int y_dtype,
                       int64_t T, int64_t k, const ccq_fp8row_experts* ex, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ccq_moe_fp8row_ffn with the shared expert's output shared [T, H] f32
 * added in the combine's epilogue as ccq_moe_combine_shared does
 * (experts/pipeline.py:181-190, blocks/moe.py:177-179). */
int ccq_moe_fp8row_ffn_shared(const float* x, const int64_t* ids, const float* weights,
                              const float* shared, float shared_gate, void* y, int y_dtype, int64_t T,
                              int64_t k, const ccq_fp8row_experts* ex, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Float32 products on already-float32 operands (fp32 MFMA: float32
 * products, float32 accumulation, operands never rounded)
 * ---------------------------------------------------------------------- */

/* Workspace bytes ccq_f32_gemm can use to split K when the output has too
 * few 64 x 64 tiles to fill the GPU (0: no split for this shape). */
size_t ccq_f32_gemm_workspace_size(int64_t M, int64_t K, int64_t N);

/* y [M, N] = x [M, K] @ w^T for w [N, K] (trans_w = 1: the router
 * x @ gate_w.T, experts/pipeline.py:145) or x @ w for w [K, N]
 * (trans_w = 0: the products of expert_ffn, blocks/moe.py:137-141).
 * Row-major, leading dimensions = row lengths; any shape (16-byte loads
 * when K, N and the pointers allow).  With the workspace of
 * ccq_f32_gemm_workspace_size, small outputs split K over workgroups and
 * add the partial sums in split order (deterministic); workspace may be
 * null (no split). */
int ccq_f32_gemm(const float* x, const float* w, float* y, int64_t M, int64_t K, int64_t N, int trans_w,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of ccq_expert_ffn_f32 (the [rows, inter] intermediate). */
size_t ccq_expert_ffn_f32_workspace_size(int64_t rows, int64_t inter);

/* expert_ffn on float32 weights (blocks/moe.py:122-141): y [rows, hidden] =
 * (silu(x @ w_gate) * (x @ w_up)) @ w_down with w_gate / w_up [hidden,
 * inter], w_down [inter, hidden]; the SiLU product in float64, rounded once
 * (silu_mul_fused, quant/kernels.py:219-231).  Two launches (gate/up with
 * the SiLU epilogue, down). */
int ccq_expert_ffn_f32(const float* x, const float* w_gate, const float* w_up, const float* w_down, float* y,
                       int64_t rows, int64_t hidden, int64_t inter, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Workspace bytes of ccq_moe_f32_ffn. */
size_t ccq_moe_f32_workspace_size(int64_t T, int64_t k, int64_t num_experts, int64_t hidden, int64_t inter);

/* moe_combine with expert_ffn over float32 expert weights found through
 * device tables of E pointers each (w_gate[e], w_up[e] [hidden, inter],
 * w_down[e] [inter, hidden]; every pointer 16-byte aligned; a null entry
 * makes that expert's rows zero): the assignments grouped by expert
 * (ccq_moe_align, 64-row tiles), one grouped gate/up launch with the SiLU
 * epilogue and one grouped down launch over all experts, then the weighted
 * combine in slot order with shared_gate * shared added when shared is not
 * null.  x [T, hidden] f32, ids [T, k] (outside [0, E): left out),
 * weights [T, k] f32, y [T, hidden] of y_dtype.  Replaces the per-expert
 * loop of moe_combine (blocks/moe.py:144-174) and of ExpertPipeline.step
 * (experts/pipeline.py:155-190) for readers that hand over float32 slots. */
int ccq_moe_f32_ffn(const float* x, const int64_t* ids, const float* weights,
                    const float* const* w_gate, const float* const* w_up, const float* const* w_down,
                    const float* shared, float shared_gate, void* y, int y_dtype, int64_t T, int64_t k,
                    int64_t num_experts, int64_t hidden, int64_t inter, void* workspace,
                    size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CCQ_H_ */

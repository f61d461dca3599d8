/*
 * biops.h -- C ABI of libbiops.so, the MI355X (gfx950) batch-invariant operator library.
 *
 * Every entry point takes raw device pointers, element strides and a hipStream_t (passed as
 * void*), launches asynchronously on that stream and returns a status code (BIOPS_OK == 0).
 * On failure biops_last_error() returns a message for the calling thread.  No entry point
 * allocates device memory: scratch space (attention scores, MoE intermediates, work lists) is
 * passed in by the caller, sized by the matching *_workspace_size() query, except for
 * biops_moe_sparse_noalloc, whose scratch is a static device array of the library.
 *
 * Batch invariance contract: for every entry point, the arithmetic that produces one output
 * element (the K-reduction order and MFMA instruction of a GEMM, the reduction tree of a row
 * reduction) depends only on the sizes of that element's own reduction (K, or the row length),
 * the dtype and the weight-side sizes (N, K), never on M, the batch count or the position of
 * the row inside the batch.
 *
 * Reference interfaces replaced (yiannisha/robotics-batch-invariant-ops, Python + Triton):
 *   batch_invariant_ops/batch_invariant_ops.py  and  batch_invariant_ops/moe.py
 * The reference has no native FFI; each function below replaces one of its Triton launch
 * wrappers (L1) or Python composites (L2), cited per declaration.
 */
#ifndef BIOPS_H
#define BIOPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (dtype arguments). */
enum {
  BIOPS_F32 = 0,
  BIOPS_F16 = 1,
  BIOPS_BF16 = 2,
  BIOPS_BOOL = 3, /* attention masks only (1 byte, nonzero = keep) */
};

/* Status codes. */
enum {
  BIOPS_OK = 0,
  BIOPS_ERR_ARG = 1,    /* invalid size / pointer / flag                           */
  BIOPS_ERR_LAYOUT = 2, /* stride pattern the kernels do not take (copy it first)  */
  BIOPS_ERR_DTYPE = 3,  /* unsupported element type                                */
  BIOPS_ERR_HIP = 4,    /* HIP runtime error (launch failure, no device)           */
  BIOPS_ERR_SIZE = 5,   /* workspace too small                                     */
};

/* Reduction operators for biops_reduce. */
enum { BIOPS_REDUCE_MEAN = 0, BIOPS_REDUCE_L2 = 1 };

/* Causal alignment for attention. */
enum {
  BIOPS_CAUSAL_NONE = 0,
  BIOPS_CAUSAL_TOP_LEFT = 1,     /* key j visible from query i iff j <= i               */
  BIOPS_CAUSAL_BOTTOM_RIGHT = 2, /* key j visible iff j <= i + (kv_len - q_len)         */
};

/* ---------------------------------------------------------------- library / device ---- */

/* Library version string ("0.2.0-mi355x"). */
const char* biops_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* biops_last_error(void);

/* Number of compute units of the current HIP device (cached per device); <0 on error.
 * Replaces get_compute_units() (batch_invariant_ops.py:232-253). */
int biops_compute_units(void);

/* ---------------------------------------------------------------------- GEMM / BMM ---- */

/* C[M,N] = A[M,K] . B[K,N] (+ bias[N]), fp32 accumulation, one rounding to dtype at the end,
 * bias added to the fp32 accumulator before that rounding.  Strides are in elements.
 * Layout: sAk == 1 (rows of A contiguous in K); either sBk == 1 (B given as W^T, the
 * nn.Linear case) or sBn == 1 (row-major B); sCn == 1.  bias may be NULL.
 * Replaces matmul_persistent + matmul_kernel_persistent (batch_invariant_ops.py:60-139,
 * 271-343) and the mm/addmm/linear shims (1600-1616). */
int biops_gemm(int dtype, int64_t M, int64_t N, int64_t K,
               const void* A, int64_t sAm, int64_t sAk,
               const void* B, int64_t sBk, int64_t sBn,
               const void* bias,
               void* C, int64_t sCm, int64_t sCn,
               void* stream);

/* Batched GEMM over a two-level batch index b = b1*nb2 + b2 (b1 < nb1, b2 < nb2):
 *   C[b] = A[b] . B[b]
 * with operand X of batch b at X + b1*sX1 + (b2/gX)*sX2, gA = gC = 1 and gB = group
 * (grouped-query attention maps gB query heads onto one key/value head; use 1 otherwise).
 * Batch strides may be 0 (broadcast operands, e.g. the MoE token matrix).  Each batch element
 * is an independent GEMM with the biops_gemm arithmetic.  Same layout rules as biops_gemm.
 * Replaces bmm_persistent + bmm_kernel_persistent (batch_invariant_ops.py:142-229, 346-431). */
int biops_bmm(int dtype, int64_t nb1, int64_t nb2, int64_t M, int64_t N, int64_t K,
              const void* A, int64_t sA1, int64_t sA2, int64_t sAm, int64_t sAk,
              const void* B, int64_t sB1, int64_t sB2, int64_t gB, int64_t sBk, int64_t sBn,
              void* C, int64_t sC1, int64_t sC2, int64_t sCm, int64_t sCn,
              void* stream);

/* dst[rows_out, cols_out] (row pitch cols_out) = src[rows, cols] (row pitch ld_src, unit
 * stride along a row), zero where r >= rows or c >= cols; rows_out >= rows, cols_out >= cols,
 * cols_out * element size a multiple of 16 bytes, dst 16-byte aligned.  Operand staging for
 * GEMMs whose K is not a whole number of 128-byte steps or whose rows are not 16-byte aligned:
 * zero-padding K changes no product bit (out-of-range K is zero in both operands on every load
 * path), and the padded operands take the direct global->LDS loads.  No counterpart in the
 * reference, whose masked Triton loads need no such copy. */
int biops_pad_rows(int dtype, int64_t rows, int64_t cols, const void* src, int64_t ld_src,
                   int64_t rows_out, int64_t cols_out, void* dst, void* stream);

/* Workspace bytes biops_gemm_padded needs for an M x N x K product whose B has strides
 * (sBk, sBn); -1 for an unsupported dtype or layout.  No counterpart in the reference. */
int64_t biops_gemm_padded_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int64_t sBk, int64_t sBn);

/* biops_gemm (same arguments and bits) on zero-padded copies of A and B written into
 * `workspace` (256-byte aligned, biops_gemm_padded_workspace_size bytes): K rounded up to a
 * whole number of 128-byte steps, rows 16-byte aligned, so that every tile entry loads the
 * operands straight into LDS.  For products whose K is not such a multiple or whose rows are
 * misaligned and which are large enough to repay two copies.  No counterpart in the reference. */
int biops_gemm_padded(int dtype, int64_t M, int64_t N, int64_t K,
                      const void* A, int64_t sAm, int64_t sAk,
                      const void* B, int64_t sBk, int64_t sBn,
                      const void* bias,
                      void* C, int64_t sCm, int64_t sCn,
                      void* workspace, int64_t workspace_bytes,
                      void* stream);

/* biops_bmm_padded_workspace_size / biops_bmm_padded: the same for a batch of independent
 * products C[b] = A[b] . B[b] (b < batch; batch strides sA, sB, sC in elements, 0 for an
 * operand shared by every batch element, which is then copied once).  Same bits as biops_bmm
 * with nb2 = gB = 1.  No counterpart in the reference. */
int64_t biops_bmm_padded_workspace_size(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                                        int64_t sA, int64_t sB, int64_t sBk, int64_t sBn);
int biops_bmm_padded(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                     const void* A, int64_t sA, int64_t sAm, int64_t sAk,
                     const void* B, int64_t sB, int64_t sBk, int64_t sBn,
                     void* C, int64_t sC, int64_t sCm, int64_t sCn,
                     void* workspace, int64_t workspace_bytes,
                     void* stream);

/* Number of entries in the GEMM tile menu.  Each entry is a (block tile, wavefront layout, LDS
 * ring depth) scheduling choice; all entries compute every output element with the same MFMA
 * sequence, so they produce identical bits and differ in speed only.  No reference
 * counterpart (the reference fixes one Triton config per dtype, batch_invariant_ops.py:294-319). */
int biops_gemm_tile_count(void);

/* Force GEMM tile entry `cfg` for every later GEMM/BMM launch in the process (-1 restores the
 * automatic choice, which is the default; the BIOPS_GEMM_CFG environment variable sets the
 * initial value).  Entries 0, 7 and 9 have no fp32 kernel and fall back to the automatic
 * choice for fp32; entries 12 (one 32x32 block per workgroup with loader wavefronts, for few
 * rows) and 13-19 (blocks of 256x256, 256x128, 128x256, 128x128, 128x64, 64x128 and 64x64 on
 * four wavefronts, 16-bit types only) need K-major B, 16-byte aligned rows and K a multiple of
 * 128 bytes and fall back to the automatic choice elsewhere.  Entries 20-22 (the
 * weight-streaming tile: 16-, 32- or 64-row m-tiles x 64 output columns, for grouped rows with few
 * rows per group) serve only the MoE expert GEMMs with 16-bit N-major weights, 16-byte aligned
 * rows and K a multiple of 128 bytes, and fall back to the automatic choice elsewhere.
 * For tuning and for the cross-entry bitwise tests.  No reference counterpart. */
int biops_set_gemm_tile(int cfg);

/* --------------------------------------------------------------- row reductions ---- */

/* out[r, :] = softmax(in[r, :]) (log_softmax if is_log != 0) over `cols` contiguous elements
 * per row, rows at stride ld_in / ld_out.  fp32 arithmetic; softmax of an all -inf row is 0.
 * dtype_in / dtype_out in {F32, F16, BF16}.
 * Replaces _softmax_kernel/softmax (batch_invariant_ops.py:1074-1145) and
 * _log_softmax_kernel/log_softmax (974-1071). */
int biops_softmax(int dtype_in, int dtype_out, int64_t rows, int64_t cols,
                  const void* in, int64_t ld_in, void* out, int64_t ld_out,
                  int is_log, void* stream);

/* Reduction over N of the strided (M, N, K) view in[m*sM + n*sN + k*sK]:
 *   MEAN: out = (sum_n x) / N       L2: out = sqrt(sum_n x*x)
 * fp32 accumulation; out[m*K + k] in dtype_out.
 * Replaces mean_kernel/mean_dim (batch_invariant_ops.py:1347-1482) and
 * _vector_norm_kernel/linalg_vector_norm_batch_invariant (1485-1597). */
int biops_reduce(int op, int dtype_in, int dtype_out, int64_t M, int64_t N, int64_t K,
                 const void* in, int64_t sM, int64_t sN, int64_t sK,
                 void* out, void* stream);

/* ---------------------------------------------------------------- convolution ---- */

/* Workspace bytes for biops_conv (same arguments; -1 for invalid sizes, 0 when none is needed). */
int64_t biops_conv_workspace_size(int dtype, int nd, int transposed, int64_t batch, int64_t cin,
                                  const int64_t* in_size, int64_t cout, const int64_t* ksize,
                                  const int64_t* stride, const int64_t* padding,
                                  const int64_t* dilation, int64_t groups);

/* nd-dimensional convolution (nd = 1, 2, 3), x[B, C_in, *in_size] with element strides
 * x_strides[nd + 2], out[B, C_out, *out_size] contiguous, bias[C_out] or NULL.  The size arrays
 * hold nd host values.
 * Regular (transposed = 0): weight [C_out, C_in/groups, *ksize] contiguous, out_size =
 * (in + 2 pad - dil (k - 1) - 1) / stride + 1.  Depthwise 1-D (groups = C_in = C_out):
 * fp32 sum over the taps in order plus the bias, one rounding.  Otherwise each output element
 * is one fixed-schedule GEMM dot product over (channel, taps) of the group, rounded, then
 * round(value + bias[c]).
 * Transposed (transposed = 1): stride == ksize, padding 0, dilation 1 only (non-overlapping);
 * weight [C_in, C_out/groups, *ksize] contiguous, out_size = in * ksize, spatial input dims
 * contiguous; one GEMM dot product over the group's input channels per output, rounded, then
 * round(value + bias[c]).
 * Replaces depthwise_conv1d_kernel and conv1d/conv2d/conv3d_batch_invariant
 * (batch_invariant_ops.py:434-780), conv_transpose2d/3d_batch_invariant (783-941) and their
 * dispatcher convolution_batch_invariant (944-971). */
int biops_conv(int dtype, int nd, int transposed, int64_t batch, int64_t cin, const int64_t* in_size,
               int64_t cout, const int64_t* ksize, const int64_t* stride, const int64_t* padding,
               const int64_t* dilation, int64_t groups,
               const void* x, const int64_t* x_strides, const void* weight, const void* bias,
               void* out, void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------- attention ---- */

/* 1 when biops_sdpa_fused takes this dtype and head sizes: bf16 or fp16, 1 <= d, dv <= 256,
 * both multiples of 8; 0 otherwise.  biops_varlen_fused_supported: the same for
 * biops_varlen_sdpa_fused, with d, dv <= 128.  No reference counterpart (the reference has one
 * eager path); callers pick the fused or the materialised entry with them. */
int biops_attention_fused_supported(int dtype, int64_t d, int64_t dv);
int biops_varlen_fused_supported(int dtype, int64_t d, int64_t dv);

/* 1 when biops_sdpa_fused takes this attention mask: unit stride between keys, batch / head /
 * query strides multiples of 4, lk a multiple of 4 and the base aligned to four elements (the
 * kernel reads four keys at once); 0 otherwise.  No reference counterpart. */
int biops_attention_fused_mask_ok(const void* mask, int mask_dtype, int64_t lk, int64_t mB, int64_t mH,
                                  int64_t mI, int64_t mJ);

/* Same operator and arguments as biops_sdpa, without a score matrix in memory and without a
 * workspace: each 128-row query tile walks 64-key blocks in order twice (row max and sum, then
 * P V), with the roundings of the eager composite (S, S*scale, S+mask and the normalised P
 * rounded to dtype).  S is bitwise the materialised S; the row sum may differ from the row
 * kernel's in the last fp32 bits.  Needs biops_attention_fused_supported, 16-byte aligned q/k/v
 * and strides that are multiples of 8 elements, and a mask (if any) that
 * biops_attention_fused_mask_ok accepts (BIOPS_ERR_LAYOUT otherwise).
 * Replaces scaled_dot_product_attention_batch_invariant (batch_invariant_ops.py:1148-1213). */
int biops_sdpa_fused(int dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk,
                     int64_t d, int64_t dv,
                     const void* q, int64_t sqB, int64_t sqH, int64_t sqL,
                     const void* k, int64_t skB, int64_t skH, int64_t skL,
                     const void* v, int64_t svB, int64_t svH, int64_t svL,
                     const void* mask, int mask_dtype, int64_t mB, int64_t mH, int64_t mI, int64_t mJ,
                     int causal, float scale, void* out, void* stream);

/* Tile order of biops_varlen_sdpa_fused: writes plan[5] entries (the plan's count of 128-row
 * query tiles) into the host array `order`, one per (sequence, query tile), as
 * (item << 32) | tile, sorted by the number of keys the tile sees under `causal`, most first
 * (ties in plan order), and returns the count, or <0 on a malformed plan.  The order only
 * schedules work: every tile's bits are the same in any order.  No reference counterpart (the
 * reference launches one eager SDPA per sequence). */
int64_t biops_varlen_fused_order(const int64_t* plan, int causal, int64_t* order);

/* Packed varlen attention with the fused kernel: same arguments as biops_varlen_sdpa without
 * the workspace (the plan from biops_varlen_plan; biops_varlen_fused_supported), plus `dorder`,
 * the device copy of biops_varlen_fused_order's array for the same plan and causal mode.  out
 * rows outside every sequence are not written.  Same layout conditions as biops_sdpa_fused.
 * Replaces varlen_scaled_dot_product_attention_batch_invariant (batch_invariant_ops.py:1216-1344). */
int biops_varlen_sdpa_fused(int dtype, int64_t hq, int64_t hkv, int64_t d, int64_t dv,
                            const void* q, int64_t sq_t, int64_t sq_h,
                            const void* k, int64_t sk_t, int64_t sk_h,
                            const void* v, int64_t sv_t, int64_t sv_h,
                            void* out, int64_t so_t, int64_t so_h,
                            const int64_t* dplan, const int64_t* hplan, const int64_t* dorder,
                            int causal, float scale, void* stream);

/* biops_varlen_plan, biops_varlen_fused_order, the upload of both and biops_varlen_sdpa_fused in
 * one call, for callers holding the offsets on the host (the reference reads them there too,
 * batch_invariant_ops.py:1264-1265): cu_q / cu_kv are host arrays of nseq + 1 offsets (starting
 * at zero, nondecreasing, within total_q query rows of q and out and total_kv key rows of k and
 * v, as the reference requires; BIOPS_ERR_ARG otherwise); host_buf (host_words int64, pinned host memory the caller
 * leaves untouched until the upload has run on `stream`) receives the plan followed by the tile
 * order, and dev_buf (device, as many words) their copy.  Rows of out outside every sequence,
 * and rows of sequences without keys, are zeroed first.  Returns BIOPS_ERR_ARG (message in
 * biops_last_error) for rejected offsets, BIOPS_ERR_SIZE when host_words is below
 * biops_varlen_plan_len(nseq) plus the plan's query-tile count; otherwise as
 * biops_varlen_sdpa_fused.  Replaces varlen_scaled_dot_product_attention_batch_invariant
 * (batch_invariant_ops.py:1216-1344) from its offsets on. */
int biops_varlen_sdpa_fused_planned(int dtype, int64_t hq, int64_t hkv, int64_t d, int64_t dv,
                                    const void* q, int64_t sq_t, int64_t sq_h,
                                    const void* k, int64_t sk_t, int64_t sk_h,
                                    const void* v, int64_t sv_t, int64_t sv_h,
                                    void* out, int64_t so_t, int64_t so_h, int64_t total_q,
                                    int64_t total_kv, int64_t nseq, const int64_t* cu_q, const int64_t* cu_kv,
                                    int64_t* host_buf, int64_t host_words, int64_t* dev_buf,
                                    int causal, float scale, void* stream);

/* Workspace bytes biops_sdpa needs (the materialised score/probability matrices). */
int64_t biops_sdpa_workspace_size(int dtype, int64_t batch, int64_t hq, int64_t lq, int64_t lk);

/* Eager attention out = softmax(round(round(Q K^T) * scale) (+mask | causal)) V with the
 * roundings of the reference composite, for Q[B,Hq,Lq,D], K[B,Hkv,Lk,D], V[B,Hkv,Lk,Dv],
 * out[B,Hq,Lq,Dv] (strides given per dim, last dim contiguous; out contiguous).  Hq must be a
 * multiple of Hkv (GQA: query head h reads key/value head h / (Hq/Hkv)).
 * mask (may be NULL): dtype BOOL (nonzero = keep) or `dtype` (additive), indexed as
 * mask[b*mB + h*mH + i*mI + j*mJ] (broadcast dims have stride 0).  causal: BIOPS_CAUSAL_*
 * (TOP_LEFT is the reference's is_causal); mask and causal are exclusive.
 * Fully masked rows give 0.
 * Replaces scaled_dot_product_attention_batch_invariant (batch_invariant_ops.py:1148-1213). */
int biops_sdpa(int dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk,
               int64_t d, int64_t dv,
               const void* q, int64_t sqB, int64_t sqH, int64_t sqL,
               const void* k, int64_t skB, int64_t skH, int64_t skL,
               const void* v, int64_t svB, int64_t svH, int64_t svL,
               const void* mask, int mask_dtype, int64_t mB, int64_t mH, int64_t mI, int64_t mJ,
               int causal, float scale,
               void* out, void* workspace, int64_t workspace_bytes, void* stream);

/* Host-side planning for packed variable-length attention.  Given the host copies of the
 * cumulative offsets (nseq+1 entries each, validated by the caller), writes the per-sequence
 * work list used by biops_varlen_sdpa into `plan` (host int64 array of
 * biops_varlen_plan_len(nseq) entries) and returns the workspace bytes needed, or <0 on a
 * malformed offset list.  Empty query or key ranges are dropped (their rows stay zero).
 * Header words: items, QK tiles, PV tiles, score rows, score elements, 128-row query tiles. */
int64_t biops_varlen_plan_len(int64_t nseq);
int64_t biops_varlen_plan(int64_t nseq, const int64_t* cu_q, const int64_t* cu_kv,
                          int64_t hq, int64_t dv, int dtype, int64_t* plan);

/* Packed varlen attention for q[1,Tq,Hq,D], k[1,Tk,Hkv,D], v[1,Tk,Hkv,Dv], out[1,Tq,Hq,Dv]
 * (token stride sX_t, head stride sX_h, last dim contiguous).  `dplan` is the device copy of
 * the host plan above; the caller has zeroed `out` (rows of no sequence stay 0).
 * causal: BIOPS_CAUSAL_NONE / TOP_LEFT / BOTTOM_RIGHT (for equal lengths both equal standard
 * causal).  Each sequence is an independent problem: its bits do not depend on the others.
 * Replaces varlen_scaled_dot_product_attention_batch_invariant (batch_invariant_ops.py:1216-1344). */
int biops_varlen_sdpa(int dtype, int64_t hq, int64_t hkv, int64_t d, int64_t dv,
                      const void* q, int64_t sq_t, int64_t sq_h,
                      const void* k, int64_t sk_t, int64_t sk_h,
                      const void* v, int64_t sv_t, int64_t sv_h,
                      void* out, int64_t so_t, int64_t so_h,
                      const int64_t* dplan, const int64_t* hplan, int causal, float scale,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------- MoE ---- */

/* Workspace bytes for biops_moe. */
int64_t biops_moe_workspace_size(int dtype, int64_t tokens, int64_t experts, int64_t hidden,
                                 int64_t inter);

/* Deterministic top-k SwiGLU mixture of experts:
 *   act[e,t,:]  = round(round(silu(round(x_t . gate_e^T))) * round(x_t . up_e^T))
 *   y[e,t,:]    = round(act[e,t,:] . down_e^T)
 *   out[t,:]    = sum over slots s = 0..k-1, left to right, each term round(y[sel[t,s],t,:] *
 *                 round(w[t,s])) and each partial sum rounded to dtype
 * x[T,D] (row stride sx), gate/up given as [E,I,D] views with strides (sgE, sgI, sgD) and
 * (suE, suI, suD), down as [E,D,I] with (sdE, sdD, sdI); each needs its D (resp. I) stride or
 * its I (resp. D) stride equal to 1.  weights[T,k] in any float dtype w_dtype (each weight is
 * rounded to dtype before the multiply, round(w[t,s]) above), sel[T,k] int64.
 * Expert indices outside [0,E) make the call write zeros for that token and set *bad_index
 * (device int32, may be NULL) to 1; the flag is never cleared by the library, so one word can
 * collect the reports of many calls until the caller reads and clears it.  out[T,D] contiguous.
 * Replaces deterministic_token_choice_moe (moe.py:11-92). */
int biops_moe(int dtype, int64_t tokens, int64_t experts, int64_t hidden, int64_t inter,
              int64_t top_k,
              const void* x, int64_t sx,
              const void* gate, int64_t sgE, int64_t sgI, int64_t sgD,
              const void* up, int64_t suE, int64_t suI, int64_t suD,
              const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
              const void* weights, int w_dtype, const int64_t* sel,
              void* out, int32_t* bad_index,
              void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes for biops_moe_sparse (-1 for experts > 2048 or invalid sizes).  About
 * tokens*top_k*(hidden + inter) elements plus small route tables. */
int64_t biops_moe_sparse_workspace_size(int dtype, int64_t tokens, int64_t top_k, int64_t experts,
                                        int64_t hidden, int64_t inter);

/* The same operator as biops_moe, same arguments and bit-identical output, evaluating only the
 * selected routes: routes t*k+s are packed by expert (ranks from wavefront ballots, no atomics),
 * each expert's rows go through the gate/up and down GEMMs as one grouped launch each, and
 * the slot sum reads the packed rows.  k/E of the dense arithmetic.  Requires experts <= 2048
 * and a 256-byte aligned workspace of biops_moe_sparse_workspace_size bytes.
 * Replaces deterministic_token_choice_moe (moe.py:11-92) with the sparse evaluation its
 * docstring names as having the same semantics (moe.py:35-38). */
int biops_moe_sparse(int dtype, int64_t tokens, int64_t experts, int64_t hidden, int64_t inter,
                     int64_t top_k,
                     const void* x, int64_t sx,
                     const void* gate, int64_t sgE, int64_t sgI, int64_t sgD,
                     const void* up, int64_t suE, int64_t suI, int64_t suD,
                     const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
                     const void* weights, int w_dtype, const int64_t* sel,
                     void* out, int32_t* bad_index,
                     void* workspace, int64_t workspace_bytes, void* stream);

/* Size of the static device array behind biops_moe_sparse_noalloc, per GPU (64 MiB). */
#define BIOPS_MOE_NOALLOC_SCRATCH_BYTES (64LL << 20)

/* biops_moe_sparse without a workspace argument and without any allocation: the same kernels,
 * arguments (minus workspace / workspace_bytes) and bit-identical output, with the route tables
 * and packed matrices in a library-owned static device array of BIOPS_MOE_NOALLOC_SCRATCH_BYTES
 * on each GPU, held until the process ends.  No hipMalloc / hipFree or other allocating call is
 * made; the array's device address is looked up once per device (hipGetSymbolAddress, with that
 * device current).  Sizes whose biops_moe_sparse_workspace_size exceeds the array return
 * BIOPS_ERR_SIZE before any GPU work (C5 shapes -- hidden 2048, intermediate 768, top-8 -- fit up
 * to 1485 tokens).  The stream must belong to the current device.  Every call on one GPU uses
 * the same array, so the calls on one GPU are ordered on the device: each call's stream waits
 * for an event recorded after the previous call's kernels (whatever stream or host thread made
 * it; no host wait).  Under stream capture that wait and record are left out: captured calls
 * and graph replays that overlap other calls on the same GPU must be ordered by the caller.
 * Nothing in the array needs to start at zero: each call writes every table before reading it.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation). */
int biops_moe_sparse_noalloc(int dtype, int64_t tokens, int64_t experts, int64_t hidden, int64_t inter,
                             int64_t top_k,
                             const void* x, int64_t sx,
                             const void* gate, int64_t sgE, int64_t sgI, int64_t sgD,
                             const void* up, int64_t suE, int64_t suI, int64_t suD,
                             const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
                             const void* weights, int w_dtype, const int64_t* sel,
                             void* out, int32_t* bad_index, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BIOPS_H */

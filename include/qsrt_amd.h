/*
 * qsrt_amd.h -- C ABI of the MI355X (gfx950) QSRT encoder hot path.
 *
 * All pointers are device pointers unless stated otherwise; every call is
 * asynchronous on `stream` (a hipStream_t passed as void*), allocates
 * nothing, and returns 0 on success or a negative status:
 *   -1 bad argument, -2 workspace too small, -3 HIP runtime error.
 * qsrt_last_error() returns a thread-local message for the last failure.
 * The caller owns all memory.  No process-global mutable state: the LUT is
 * passed per call (unlike the reference's __constant__ table pointer,
 * qsrt/csrc/sqg_quantize.cu:14, :698-705).
 */
#ifndef QSRT_AMD_H
#define QSRT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI revision of this header. */
int qsrt_abi_version(void);

/* Message for the last failing call on this thread. */
const char *qsrt_last_error(void);

/*
 * Bytes of traceback workspace qsrt_viterbi_tiles needs for `n_tiles` tiles
 * at rate K on the current device (one 256-row decision buffer per
 * workgroup, at most one workgroup per compute unit).  0 on error.
 * Replaces the workspace sizing of qsrt/sqg_quantizer.py:410-427
 * (_sqg_temp_buffers).
 */
size_t qsrt_viterbi_workspace_bytes(int K, int64_t n_tiles);

/*
 * Tail-biting L16 trellis quantization of `n_tiles` 256-weight tiles.
 *   tiles   f32 [n_tiles, 256]  targets in tensor-core order
 *   recon   f32 [n_tiles, 256]  out: E4M3 label of each emitted codeword
 *   states  u16 [n_tiles, 256]  out: 16-bit codewords (closed cyclic path)
 *   K       1 .. 6 branch bits per weight (the reference's K1..K6 dispatch,
 *           qsrt/csrc/sqg_quantize.cu:720-780)
 *   tailbite_context  1..128 primer half-width C
 *   lut_e4m3  u8 [65536] state(codeword)-indexed E4M3 labels
 *   boundary_lag  0: boundary = argmin of the primer's final costs
 *                 1: argmin of the costs one step earlier
 *   workspace  >= qsrt_viterbi_workspace_bytes(K, n_tiles) bytes
 * FP32 path metrics, lowest-index ties (see oracle/viterbi_ref.c).
 * Replaces quantize_tiles_sqg_cuda (qsrt/csrc/sqg_quantize.cu:651-783) and
 * the kernels it launches (qsrt_quantize_tiles_kernel.cuh:26-500,
 * qsrt_quantize_tiles_k2_kernel.cuh:47-366); bound from Python where the
 * reference binds `quantize_tiles_sqg` (qsrt/csrc/sqg_quantize.cpp:56-59).
 */
int qsrt_viterbi_tiles(const float *tiles, float *recon, uint16_t *states, int64_t n_tiles, int K,
                       int tailbite_context, const uint8_t *lut_e4m3, int boundary_lag, void *workspace,
                       size_t workspace_bytes, void *stream);

/*
 * qsrt_viterbi_tiles on at most `max_workgroups` compute units (0: all of
 * them).  Two rate groups of one BlockLDLQ step launched on two streams
 * with grids in proportion to their work run side by side instead of one
 * after the other (each workgroup holds a whole CU).  The workspace needs
 * at most qsrt_viterbi_workspace_bytes(K, n_tiles) bytes.  Same results as
 * qsrt_viterbi_tiles for any grid.  No counterpart in the reference, whose
 * launcher always sizes the grid from the tile count
 * (qsrt/csrc/sqg_quantize.cu:507-576).
 */
int qsrt_viterbi_tiles_ex(const float *tiles, float *recon, uint16_t *states, int64_t n_tiles, int K,
                          int tailbite_context, const uint8_t *lut_e4m3, int boundary_lag, int max_workgroups,
                          void *workspace, size_t workspace_bytes, void *stream);

/*
 * The reference extension's call shape, argument for argument:
 * quantize_tiles_sqg(input_tiles, output_tiles, output_indices, temp_costs,
 * temp_edges, codebook, K, tailbite_context, lut_abs_max)
 * (qsrt/csrc/sqg_quantize.cpp:56-59 -> qsrt/csrc/sqg_quantize.cu:651-783),
 * with each tensor as a device pointer (and byte size for the two
 * temporaries), so the reference's own caller (qsrt/sqg_quantizer.py:
 * 478-654) binds it unchanged.  `codebook` is what that caller passes: for
 * K2..K4 its [out-edge pair][predecessor][2] transpose of the state-indexed
 * E4M3 table (qsrt/sqg_quantizer.py:612-633), otherwise the table itself.
 * The FP16 cost buffer is not needed here (costs live in LDS); its first
 * 64 KiB receive the state-indexed table.  `temp_edges` is the traceback
 * workspace and bounds how many compute units run at once.  The boundary
 * rule follows the reference's kernel choice: K2 with a finite lut_abs_max
 * in (0, 16] scores the last primer step, every other case the one before.
 * Path metrics are FP32 with lowest-index ties (the reference's are FP16).
 */
int qsrt_quantize_tiles_sqg(const float *input_tiles, float *output_tiles, int16_t *output_indices, int64_t n_tiles,
                            void *temp_costs, size_t temp_costs_bytes, uint8_t *temp_edges, size_t temp_edges_bytes,
                            const uint8_t *codebook, int K, int tailbite_context, double lut_abs_max, void *stream);

/*
 * EXL word packing of n_tiles tiles at rate K (1..6; the QSRT container uses
 * 2..4, the uniform codec paths of qsrt/qsrt_codec_pilot.py:220-281 up to 6):
 *   states u16 [n_tiles, 256] (only the low K bits are stored; 16-byte
 *   aligned), words i16 [n_tiles, 16 K] out.
 * Replaces the un-vendored ext.pack_trellis called from
 * qsrt/exl3_encoder_backend.py:2361-2372, whose word order the reference
 * restates in qsrt/qsrt.py:861-883 (pack_trellis_edges).
 */
int qsrt_pack_edges(const uint16_t *states, int64_t n_tiles, int K, int16_t *words, void *stream);

/*
 * Inverse of qsrt_pack_edges followed by the cyclic state closed form:
 *   words i16 [n_tiles, 16 K] -> states u16 [n_tiles, 256], K 1..6.
 * Replaces unpack_trellis_states (qsrt/qsrt.py:910-913) =
 * unpack_trellis_edges (:886-907) + reconstruct_trellis_states
 * (qsrt/exl3_reference.py:34-58).
 */
int qsrt_unpack_states(const int16_t *words, int64_t n_tiles, int K, uint16_t *states, void *stream);

/*
 * Blockwise normalised Sylvester-Hadamard rotation, in place, of an FP32
 * row-major matrix x [rows, cols] with leading dimension ld (elements):
 *   side 0: each group of `block` rows  r  ->  H_block @ r
 *   side 1: each group of `block` cols  c  ->  c @ H_block
 * H_block[i][j] = (-1)^popcount(i & j) / sqrt(block); block 64..512.
 * Optional device vectors of length rows (side 0) or cols (side 1), NULL
 * for none, fuse the surrounding scalings:
 *   x[a] <- post_mul[a] * H(x * pre_mul / pre_div)[a].
 * x 16-byte aligned; cols and ld multiples of 4.
 * Replaces preapply_had_l/_r and blockwise_preapply_had_l_/_r_
 * (qsrt/exl3_encoder_backend.py:275-320) and block_hadamard /
 * signed_block_hadamard (qsrt/qsrt_coupled.py:49-126).
 */
int qsrt_hadamard(float *x, int64_t rows, int64_t cols, int64_t ld, int block, int side, const float *pre_mul,
                  const float *pre_div, const float *post_mul, void *stream);

/*
 * qsrt_hadamard on a float64 matrix with float64 vectors (x 16-byte
 * aligned, cols and ld multiples of 4).  The encoder's regularisation
 * rotates in float64 (W / sv, then H; W / su, then H on the other side) so
 * that the weight the BlockLDLQ recursion reads is rounded to FP32 only in
 * the tile targets.  Replaces the same reference functions as qsrt_hadamard
 * on the regularize path (qsrt/exl3_encoder_backend.py:2580-2708, which
 * rotates in FP32).
 */
int qsrt_hadamard_f64(double *x, int64_t rows, int64_t cols, int64_t ld, int block, int side, const double *pre_mul,
                      const double *pre_div, const double *post_mul, void *stream);

/*
 * One matrix (or a run of record strips of a mixed-rate matrix) for
 * qsrt_decode.  The matrix is a grid of 128 x 128 blocks of 8 x 8 tiles;
 * tile (i, j) of block (R, C) starts at
 *   words + R * block_row_stride + C * block_col_stride
 *         + i * tile_row_stride + j * tile_col_stride      (int16 elements)
 * (block strides of 0 mean 8 * tile_row_stride and 8 * tile_col_stride: a
 * plain tile grid) and holds 16 K int16 EXL words.  Output element (r, c)
 * is written to
 *   out[r * out_ld + c] = row_scale[r] * col_scale[c] * (H X H)[r][c]
 * with H the unnormalised 128-block +-1 Sylvester Hadamard (pass
 * row_scale = su / 128 to reproduce the normalised decode).
 */
typedef struct qsrt_decode_job {
    const int16_t *words;
    int64_t tile_row_stride;
    int64_t tile_col_stride;
    const float *row_scale;
    const float *col_scale;
    void *out;
    int64_t out_ld;
    int64_t rows;
    int64_t cols;
    int64_t block_row_stride;
    int64_t block_col_stride;
} qsrt_decode_job;

/* Device workspace bytes qsrt_decode needs for n_jobs jobs. */
size_t qsrt_decode_workspace_bytes(int n_jobs);

/*
 * Fused decode of packed trellis payloads at rate K (2..4) to bf16
 * (out_dtype 0) or f32 (out_dtype 1):
 *   words -> cyclic 16-bit states -> lut_e4m3[state] -> X (tensor-core
 *   order inside each 16x16 tile) -> row_scale . H128 X H128 . col_scale.
 * `jobs` is a HOST array, written into `workspace` by a stream-ordered
 * upload kernel whose arguments carry the jobs (no host staging buffer, no
 * allocation; `jobs` may be reused as soon as the call returns); rows and cols
 * multiples of 128; words, out, row_scale and col_scale 16-byte aligned;
 * tile and block strides multiples of 8; out_ld >= cols and a multiple of 8; lut_e4m3
 * 16-byte aligned.  exact_fp8 != 0 selects the FP8 matrix-core path, exact
 * for LUTs with |label| <= 6 (every SQG table); 0 the FP32 path (any LUT).
 * Equivalent to qsrt_decode_prepare followed by qsrt_decode_execute.
 * Replaces decode_exl3_weight / decode_qsrt_weight
 * (qsrt/exl3_reference.py:61-330) and decode_qsrt_exl3_weight
 * (qsrt/qsrt.py:1175-1209).
 */
int qsrt_decode(const qsrt_decode_job *jobs, int n_jobs, int K, const uint8_t *lut_e4m3, int exact_fp8,
                int out_dtype, void *workspace, size_t workspace_bytes, void *stream);

/*
 * A validated job table resident in a caller's workspace: decode the same
 * set of payloads many times (a serving layer, a benchmark) without
 * re-validating or re-uploading it.  Plain data: copy it freely; it stays
 * valid while the workspace and every pointer in the jobs do.
 */
typedef struct qsrt_decode_plan {
    const void *jobs;     /* device job table inside the workspace */
    int n_jobs;           /* non-empty jobs */
    int K;
    int64_t total_blocks; /* 128 x 128 blocks over all jobs */
} qsrt_decode_plan;

/* Validate `jobs` (same rules as qsrt_decode) and upload them into
 * `workspace` on `stream`; fills *plan. */
int qsrt_decode_prepare(const qsrt_decode_job *jobs, int n_jobs, int K, void *workspace, size_t workspace_bytes,
                        qsrt_decode_plan *plan, void *stream);

/* One launch over a prepared plan (stream-ordered after its upload). */
int qsrt_decode_execute(const qsrt_decode_plan *plan, const uint8_t *lut_e4m3, int exact_fp8, int out_dtype,
                        void *stream);

/*
 * qsrt_decode with no workspace argument and no allocation of any kind: the
 * job table lives in the library's own device array (`scratch` in decode.hip,
 * 4096 jobs = 352 KiB, held by each GPU the library runs on until the process
 * ends) and is written by a stream-ordered upload kernel, so the call issues
 * only kernel launches.  Same arguments, validation and results as
 * qsrt_decode; n_jobs > 4096 is rejected (-1).  Every call on one GPU shares
 * that GPU's table, so calls that overlap on one GPU (different streams or
 * threads without ordering) race; calls ordered on one stream do not.
 * No counterpart in the reference: it exists for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).
 */
int qsrt_decode_noalloc(const qsrt_decode_job *jobs, int n_jobs, int K, const uint8_t *lut_e4m3, int exact_fp8,
                        int out_dtype, void *stream);

/*
 * C[M, N] += alpha * A^T (B - B2) on the matrix cores, all row-major:
 *   A [K, M] (lda), B and B2 [K, N] (ldb), C [M, N] f32 (ldc).
 *   dtype 0: f32 operands (16-byte aligned, lda/ldb multiples of 4), exact
 *            FP32 products; B2 may be NULL (no subtraction).
 *   dtype 1: bf16 operands (raw uint16 bits), FP32 accumulation; B2 NULL.
 * Replaces the BlockLDLQ feedback products prod_cache += L^T (W - Q)
 * (qsrt/exl3_encoder_backend.py:496, :534; batched :1170-1187) and the
 * Hessian capture H += X^T X.
 */
int qsrt_gemm_tn(float *C, const void *A, const void *B, const void *B2, int64_t M, int64_t N, int64_t K,
                 int64_t lda, int64_t ldb, int64_t ldc, float alpha, int dtype, void *stream);

/*
 * Device bytes qsrt_gemm_tn_ws wants as workspace for these arguments (0 when
 * the call has nothing to split: dtype 0, or a bf16 tile count that fills the
 * device's compute units in whole rounds).
 */
size_t qsrt_gemm_tn_workspace_bytes(const float *C, const void *A, const void *B, int64_t M, int64_t N, int64_t K,
                                    int64_t lda, int64_t ldb, int64_t ldc, int dtype);

/*
 * qsrt_gemm_tn with a device workspace (16-byte aligned).  bf16: when the
 * 256 x 256 tiles do not fill the compute units in whole rounds, the tiles of
 * the last round are split along K and their partial products, written to
 * the workspace, are added to C in K order by a second kernel on the same
 * stream (the result is deterministic; it differs from the unsplit sum only
 * by FP32 rounding).  A NULL or short workspace runs every tile whole, as
 * qsrt_gemm_tn does.  Same operator and call sites as qsrt_gemm_tn.
 */
int qsrt_gemm_tn_ws(float *C, const void *A, const void *B, const void *B2, int64_t M, int64_t N, int64_t K,
                    int64_t lda, int64_t ldb, int64_t ldc, float alpha, int dtype, void *workspace,
                    size_t workspace_bytes, void *stream);

/*
 *   C[M, N] += alpha * A^T (B - B2)      A: [K, M] f64, B: [K, N] f64,
 *                                        B2: [K, N] f32 or NULL, C: [M, N] f64
 * row-major with leading dimensions lda, ldb, ldb2, ldc (elements; even).
 * A and B 16-byte aligned.  Float64 matrix cores (v_mfma_f64_16x16x4_f64);
 * every element of C sums its K terms in the same order for any M and N.
 * The BlockLDLQ product-cache update P += L[span]^T (W - Q)[span] under the
 * encoder's float64 contract (factor and regularised weight float64, the
 * reconstruction FP32).  Replaces the reference's FP32 span products
 * (qsrt/exl3_encoder_backend.py:534, batched :1450-1471).
 */
int qsrt_gemm_tn_f64(double *C, const double *A, const double *B, const float *B2, int64_t M, int64_t N, int64_t K,
                     int64_t lda, int64_t ldb, int64_t ldb2, int64_t ldc, double alpha, void *stream);

/*
 * qsrt_gemm_tn_f64 over `batch` members in one launch:
 *   C[b] += alpha * A[b]^T (B[b] - B2[b])    b < batch
 * with X[b] = X + b * stride_x (elements; even, and stride_c >= (M - 1) * ldc + N
 * so the members of C do not overlap).  Each member's elements are computed
 * exactly as qsrt_gemm_tn_f64 computes them.  The batched BlockLDLQ span
 * product of the mixed and batched recursions, which the reference issues as
 * one baddbmm over the members: _baddbmm_ldlq(product_cache[:, :begin],
 * Ls[:, begin:end, :begin]^T, W[:, begin:end] - Q[:, begin:end])
 * (qsrt/exl3_encoder_backend.py:1170-1187, call :1458-1471).
 */
int qsrt_gemm_tn_f64_batched(double *C, const double *A, const double *B, const float *B2, int batch, int64_t M,
                             int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldb2, int64_t ldc, int64_t stride_c,
                             int64_t stride_a, int64_t stride_b, int64_t stride_b2, double alpha, void *stream);

/*
 * Diagonal-block step of a blocked float64 Cholesky factorisation, for
 * `batch` matrices A[b] = A + b * batch_stride (n x n, row-major, leading
 * dimension n).  The lower triangle of the nb x nb block at (j0, j0) is
 * factored in place (L11, zeros written above its diagonal) and L11^-1 is
 * written to inv[b] (nb x nb row-major, zeros above the diagonal), so the
 * caller's panel solve and trailing update are two DGEMMs.  A pivot that is
 * not positive sets info[b] (int32, device) to j0 + k + 1, the order of the
 * failing leading minor as LAPACK reports it, unless info[b] is already
 * non-zero; that block is then undefined.  nb <= 128.  Replaces the
 * factorisation inside block_ldl (qsrt/exl3_encoder_backend.py:323-393),
 * which the reference runs as torch.linalg.cholesky in FP32.
 */
int qsrt_chol_diag_block_f64(double *A, int64_t n, int64_t batch, int64_t batch_stride, int64_t j0, int nb,
                             double *inv, int32_t *info, void *stream);

/*
 * Unit block-lower factor of `batch` lower Cholesky factors, in place:
 * C[b] = C + b * batch_stride (n x n, element (i, c) at i * row_stride +
 * c * col_stride, one of the two strides 1; lower triangle holding the
 * factor, zeros above).  With 16 x 16 column blocks j, rows i >= 16 j + 16
 * become C[i, 16j:16j+16] inv[b][j], the diagonal blocks become the
 * identity and the zeros above them are kept.  inv is [batch][n / 16][16][16]
 * row-major, the inverses of the diagonal blocks.  n is a multiple of 16,
 * the leading dimension at least n, batch <= 65535; row-major matrices need
 * 16-byte aligned rows.  Replaces the column-block products and identity
 * blocks of block_ldl (qsrt/exl3_encoder_backend.py:375-390).
 */
int qsrt_block_unit_lower_f64(double *C, const double *inv, int64_t batch, int64_t n, int64_t row_stride,
                              int64_t col_stride, int64_t batch_stride, void *stream);

/*
 * One band propagation of the recursive BaKron two-sided rounding, FP32,
 * 16 x 16 blocks.  workspace (T), quantized (Q) and intermediate (I) are
 * [batch, n_out, n_in] row-major; output_factor and input_factor are
 * [n_out, n_out] and [n_in, n_in] per member at the given batch strides (0:
 * one factor shared by every member).  With block (o, i) on anti-diagonal
 * o + i, ob = n_out / 16, ib = n_in / 16 and the diagonals
 * 0 <= first < middle < last <= ob + ib - 1:
 *   I(o, i)  = sum_{s in [max(0, first - i), min(ob, middle - i))} Lout(o, s) (Q - T)(s, i)
 *              for first <= o + i < last;
 *   T(o, c) += sum_{s in [max(0, first - o), min(ib, middle, last - o))} I(o, s) Lin(c, s)^T
 *              for middle <= o + c < last.
 * Other blocks of T and I are not touched.  n_out and n_in are positive
 * multiples of 16 with n_out * n_in <= 2^31, batch <= 65535.  Replaces
 * bakron_block_update_cuda (qsrt/csrc/sqg_quantize.cu:991-1100, kernels
 * :141-270), bound as qsrt/sqg_quantizer.py:383-407.
 */
int qsrt_bakron_band_update_f32(float *workspace, const float *quantized, const float *output_factor,
                                const float *input_factor, float *intermediate, int64_t batch, int64_t n_out,
                                int64_t n_in, int64_t output_factor_batch_stride, int64_t input_factor_batch_stride,
                                int64_t first_diagonal, int64_t middle_diagonal, int64_t last_diagonal,
                                void *stream);

/*
 * qsrt_bakron_band_update_f32 for block-lower output factors (Lout(o, s) = 0
 * for every block s > o, as the unit-block-lower factors of the BaKron
 * recurrence are): the left product skips those blocks.  For such factors
 * and finite inputs the result equals qsrt_bakron_band_update_f32's (up to
 * the sign of a zero).  No counterpart in the reference, whose launcher
 * (qsrt/csrc/sqg_quantize.cu:991-1100) always takes the full ranges; for
 * callers whose factors are block-lower by construction.
 */
int qsrt_bakron_band_update_lower_f32(float *workspace, const float *quantized, const float *output_factor,
                                      const float *input_factor, float *intermediate, int64_t batch, int64_t n_out,
                                      int64_t n_in, int64_t output_factor_batch_stride,
                                      int64_t input_factor_batch_stride, int64_t first_diagonal,
                                      int64_t middle_diagonal, int64_t last_diagonal, void *stream);

/*
 * BlockLDLQ step, batched over B members (member m quantizes source
 * src[m]).  For the 16-row block [blk, blk + 16) of a span ending at row
 * `end`, every member's target
 *   T_m = W_s[blk] + mult[m] * (P_m[blk] + L_s[blk+16:end, blk:blk+16]^T (W_s - Q_m)[blk+16:end])
 * is computed in float64 and written, rounded once to FP32, one 16 x 16 tile
 * per 16 columns in tensor-core order, to tile slot[m * N/16 + t] of `tiles`
 * ([slots, 256] f32; the caller groups slots by rate).  W [S, K, N],
 * L [S, K, K] and P [B, K, N] row-major f64, Q [B, K, N] row-major f32, with
 * batch strides sW, sL, sQ, sP (elements); src int32 [B] device, mult f64 [B]
 * device, slot int32 [B * N/16] device.  K and N multiples of 16, blk a
 * multiple of 16 with blk + 16 <= end <= K.  Each element sums P first, then
 * the products in increasing row order, independent of B and N.
 * Replaces the per-step clone, product (prod_cache + L^T (W - Q)), add,
 * stack and tensor-core gather of ldlq / ldlq_mixed_batched
 * (qsrt/exl3_encoder_backend.py:420-539, :1190-1478).
 */
int qsrt_ldlq_targets(float *tiles, const double *W, const double *L, const float *Q, const double *P,
                      const int32_t *src, const double *mult, const int32_t *slot, int B, int64_t K, int64_t N,
                      int64_t sW, int64_t sL, int64_t sQ, int64_t sP, int64_t blk, int64_t end, void *stream);

/*
 * Commit of a BlockLDLQ step: rows [blk, blk + 16) of every Q_m ([B, K, N]
 * f32, batch stride sQ) take the reconstruction tiles recon[slot[m N/16 + t]]
 * (tensor-core order, f32 [slots, 256]) and tile row blk / 16 of every
 * encoded_m ([B, K/16, N/16, 256] int16, batch stride sE) the states
 * states[slot[...]] (u16 [slots, 256]).  Replaces the scatter of the
 * reconstruction and states after each tile call (reference :1055-1070,
 * :1419-1440).
 */
int qsrt_ldlq_commit(float *Q, int16_t *encoded, const float *recon, const uint16_t *states, const int32_t *slot,
                     int B, int64_t K, int64_t N, int64_t sQ, int64_t sE, int64_t blk, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QSRT_AMD_H */

/*
 * rocknpu_hip.h — device-pointer launch layer of the MI355X build.
 *
 * These entry points replace the NPU executor layer the reference's C ABI
 * drives (crates/rocknpu-matmul) and the llama.cpp CPU decode kernels the
 * reference plugin leaves M=1 to. Every pointer is a DEVICE pointer; `stream`
 * is a hipStream_t (NULL = the null stream). Calls validate their arguments on
 * the host, enqueue kernels and return without synchronising; status codes
 * are those of rocknpu.h (0 ok, -1 invalid argument, -3 launch failure).
 *
 * Device layouts: W8 is [n, k_pad] int8 row-major with k_pad a multiple of 64
 * and columns k..k_pad zero; A8 is [m, k_pad] likewise; scales are f32; Q8_K
 * rows are k/256 blocks of 292 bytes (f32 d, int8 qs[256], int16 bsums[16]).
 */
#ifndef ROCKNPU_HIP_H
#define ROCKNPU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Kernel (a): GGUF K-quant -> W8 repack. Replaces the host repack
 * prepare_q4_k_w8a8 / prepare_q5_k_w8a8 / prepare_q6_k_w8a8
 * (crates/rocknpu-capi/src/lib.rs:711-757, :759-806, :974-994) and the
 * resident weight placement of Int8DecodePool::prepare_weights_mtile_direct_with_split
 * (crates/rocknpu-matmul/src/int8_decode_pool.rs:606-615).
 * kind 4/5 need `blocks` 16-byte aligned, kind 6 2-byte aligned; w8 16-byte
 * aligned. A row whose dequantised values are not all finite gets scale NaN
 * (the reference rejects such a weight). */
int rocknpu_hip_repack_w8(uint32_t kind, const uint8_t * blocks, size_t blocks_bytes, size_t k,
                          size_t n, size_t k_pad, int8_t * w8, float * scales, void * stream);

/* Kernel (b): per-token symmetric int8 quantisation of A [m, lda] f32 (first k
 * columns) into A8 [m, k_pad]. Replaces the per-row quantize_symmetric_into
 * loop of crates/rocknpu-capi/src/lib.rs:1776-1791 (definition :614-654).
 * A row holding a non-finite value gets scale NaN and a zero int8 row. */
int rocknpu_hip_quantize_a8(const float * a, size_t m, size_t k, size_t lda, size_t k_pad,
                            int8_t * a8, float * scales, void * stream);

/* Kernel (c): out[m, ldo] = (f32(A8 W8^T) * a_scales[m]) * w_scales[n] on int8
 * MFMA; if out_i32 is non-NULL the exact int32 accumulators are also written
 * there as [m, n]. Replaces Int8DecodePool::execute_prepared_mtile_direct
 * (crates/rocknpu-matmul/src/int8_decode_pool.rs:625-686) plus the
 * rescale_i32_row sink (crates/rocknpu-capi/src/lib.rs:692-709, :1868-1884).
 * a8 and w8 16-byte aligned, k_pad a multiple of 64 and at most 133120 (the
 * largest K whose int32 sums are exact: 127 * 127 * K < 2^31). */
int rocknpu_hip_gemm_w8a8(const int8_t * a8, const float * a_scales, const int8_t * w8,
                          const float * w_scales, size_t m, size_t n, size_t k_pad, float * out,
                          size_t ldo, int32_t * out_i32, void * stream);

/* rocknpu_hip_gemm_w8a8 with a caller workspace, which lets the GEMM split
 * each tile's K range over several workgroups where its tiles would fill at
 * most half the GPU (rocknpu_hip_gemm_workspace says when, and how many bytes).
 * The split workgroups add their int32 partial tiles (exact, so the results
 * are bit-identical to the unsplit call's). The workspace is device memory,
 * 256-byte aligned, whose first 16 KiB hold the tile counters and an error
 * word, followed by the partial tiles and per-split arrival stamps: zero a
 * workspace once after allocating it, and every call that completes leaves it
 * zeroed (whatever shapes share it). A call that finds its counters not zero
 * (a workspace never zeroed, a call that did not complete, calls overlapping
 * on one workspace) writes NaN for the f32 results of the tiles concerned and
 * sets the error word, which rocknpu_hip_gemm_workspace_check reports; such a
 * workspace stays flagged until it is zeroed again. A workspace smaller than
 * the route asks for (or NULL with 0 bytes) runs the GEMM unsplit, and so does
 * a device other than gfx950 (the exchange between the split workgroups is
 * checked there only). Calls that overlap (other streams) need workspaces of
 * their own. No counterpart in the
 * reference (its NPU K-split, crates/rocknpu-capi/src/lib.rs:1885-1926, adds
 * int32 partials on the host); the product is that of rocknpu_hip_gemm_w8a8. */
int rocknpu_hip_gemm_w8a8_ws(const int8_t * a8, const float * a_scales, const int8_t * w8,
                             const float * w_scales, size_t m, size_t n, size_t k_pad, float * out,
                             size_t ldo, int32_t * out_i32, void * workspace, size_t workspace_bytes,
                             void * stream);

/* The workspace rocknpu_hip_gemm_w8a8_ws uses for an M x N x k_pad product on
 * a GPU of `cus` compute units (cus <= 0: the current device's): *bytes (0 when
 * the product runs unsplit) and the K split *splits (1: none). Host code only;
 * no GPU is needed when cus > 0. No counterpart in the reference. */
int rocknpu_hip_gemm_workspace(size_t m, size_t n, size_t k_pad, int cus, size_t * bytes, int * splits);

/* Waits for `stream`, then reads and clears the error word of a K-split
 * workspace: 0 when no call on it since the last check found dirty counters,
 * -3 (ROCKNPU_STATUS_EXECUTION_ERROR) when one did (the f32 results of its
 * affected tiles are NaN; zero the workspace before using it again), -1 for a
 * NULL workspace. No counterpart in the reference. */
int rocknpu_hip_gemm_workspace_check(void * workspace, void * stream);

/* The W8A8 GEMM on a given tile (bm x bn: 32x64 with 4 stages, k_pad % 128
 * == 0 only; 64x32 and 64x64 with 2 or 4 stages, 128x64 with 2 or 4, 128x128
 * with 2 or 3, 256x128 with 3, 256x256 with 2; bm = 0: the weight-streaming
 * kernel, m <= 16) and K split (1 to 16; above 1
 * the workspace must be a zeroed one of rocknpu_hip_gemm_w8a8_ws's layout: the
 * 16 KiB counter block, one counter per tile and at most 4095 tiles, then
 * splits x bm x bn int32 per tile, then splits x tiles stamps rounded up to
 * 256 bytes). For tests and tuning:
 * every choice gives the same bits. No
 * counterpart in the reference. */
int rocknpu_hip_gemm_w8a8_tile(int bm, int bn, int stages, int splits, const int8_t * a8,
                               const float * a_scales, const int8_t * w8, const float * w_scales, size_t m,
                               size_t n, size_t k_pad, float * out, size_t ldo, int32_t * out_i32,
                               void * workspace, size_t workspace_bytes, void * stream);

/* Kernels (b) + (c): the W8A8 prompt route on device buffers. A [m, lda] f32
 * (first k columns) is quantised per token into an int8 workspace, then
 * out[m, ldo] = (f32(A8 W8^T) * a_scale[m]) * w_scales[n] against the resident
 * W8 [n, k_pad] (16-byte aligned, k_pad a multiple of 64, at most 133120).
 * The library allocates the workspace (m * k_pad bytes + m scales, and the
 * GEMM's K-split workspace where the route splits) on `stream`, stream-ordered,
 * and releases it behind the GEMM. Replaces the
 * quantise / i32 GEMM / rescale sequence of execute_cached_w8a8_mtile_pool_padded
 * (crates/rocknpu-capi/src/lib.rs:1776-1791, :1868-1884) without its weight
 * cache. Results equal rocknpu_hip_quantize_a8 followed by rocknpu_hip_gemm_w8a8. */
int rocknpu_hip_matmul_w8a8_f32(const float * a, size_t m, size_t k, size_t lda, const int8_t * w8,
                                const float * w_scales, size_t n, size_t k_pad, float * out, size_t ldo,
                                void * stream);

/* rocknpu_hip_matmul_w8a8_f32 without allocating: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * workspace is a fixed array in the library's device memory, one copy per GPU
 * the library runs on, held until the process ends (64 KiB of scales, 32 MiB
 * of A8 and 4 MiB + 17 KiB for the GEMM's K split): at most 16384 rows and
 * m * k_pad <= 32 MiB; beyond that the call returns
 * ROCKNPU_STATUS_INVALID_ARGUMENT and prints the limit on stderr. Every call on
 * one GPU uses that GPU's copy, so calls that overlap on one GPU (other
 * streams, other threads) race. Same arguments and results as
 * rocknpu_hip_matmul_w8a8_f32. */
int rocknpu_hip_matmul_w8a8_f32_noalloc(const float * a, size_t m, size_t k, size_t lda, const int8_t * w8,
                                        const float * w_scales, size_t n, size_t k_pad, float * out,
                                        size_t ldo, void * stream);

/* The tile rocknpu_hip_gemm_w8a8 runs an M x N x k_pad product with on a GPU
 * of `cus` compute units (cus <= 0: the current device's): *bm x *bn tiles of
 * *stages 128-byte K stages, or *bm = 0 for the weight-streaming kernel of up
 * to 16 rows. Host code only; no GPU is needed when cus > 0. The choice has no
 * effect on the results, which are exact. No counterpart in the reference: its
 * NPU tiles are fixed by the register-command programs. */
int rocknpu_hip_gemm_route(size_t m, size_t n, size_t k_pad, int cus, int * bm, int * bn, int * stages);

/* Whether rocknpu_hip_gemm_w8a8 runs an M x N x k_pad product (M > 256) as two
 * launches on a GPU of `cus` compute units (cus <= 0: the current device's):
 * *n0 > 0 when the 256 x 256 tiles make one or more whole rounds plus a last
 * round at most half full; columns [0, *n0) then run on 256 x 256 tiles and
 * [*n0, N) as a product of their own (rocknpu_hip_gemm_route of M x (N - *n0)
 * x k_pad). *n0 = 0: one launch on rocknpu_hip_gemm_route's tile. Host code
 * only; the results are the same bits either way. No counterpart in the
 * reference. */
int rocknpu_hip_gemm_column_split(size_t m, size_t n, size_t k_pad, int cus, size_t * n0);

/* The launch shape rocknpu_hip_gemv_q_f32 (fused != 0) or rocknpu_hip_gemv_q8_k
 * (fused == 0) takes for `count` projections of n[i] rows, K = k and m
 * activation rows on `cus` compute units (cus <= 0: the current device's), for
 * its first launch (m beyond one launch's rows, up to 16 on the matrix-core
 * Q4_K kernel and 8 otherwise, runs in several): *mfma = 1 for the matrix-core kernel,
 * *mfma = 2 for the Q6_K kernel that streams the weights through LDS (*lanes = 8
 * lanes per super-block, *waves = its stream waves per workgroup), else 0 for
 * the lane-per-block kernel with *lanes lanes per super-block and *waves
 * waves per workgroup. Host code only; no GPU is needed when cus > 0. No
 * counterpart in the reference, whose decode GEMV runs on the CPU. */
int rocknpu_hip_gemv_shape(uint32_t kind, size_t m, size_t k, const size_t * n, size_t count, int fused, int cus,
                           int * mfma, int * lanes, int * waves);

/* Q8_K activation quantisation of x [m, ldx] f32 (k a multiple of 256) into
 * m rows of k/256 Q8_K blocks. Replaces ggml quantize_row_q8_K
 * (llama.cpp, ggml-quants.c quantize_row_q8_K_ref). q8k 4-byte aligned. */
int rocknpu_hip_quantize_q8_k(const float * x, size_t m, size_t k, size_t ldx, uint8_t * q8k,
                              void * stream);

/* Kernel (d): decode GEMV out[mi * ldo + ni] = vec_dot(W row ni, Q8_K row mi)
 * for Q4_K (kind 4, `w` 16-byte aligned) or Q6_K (kind 6, 2-byte aligned)
 * weights. Replaces ggml_vec_dot_q4_K_q8_K / ggml_vec_dot_q6_K_q8_K (llama.cpp
 * ggml-cpu). If isum/msum are non-NULL the exact per-(mi, ni, block) integer
 * sums are written there as [m][n][k/256] (msum is 0 for Q6_K). */
int rocknpu_hip_gemv_q8_k(uint32_t kind, const uint8_t * w, size_t w_bytes, size_t k, size_t n,
                          const uint8_t * q8k, size_t m, float * out, size_t ldo, int32_t * isum,
                          int32_t * msum, void * stream);

/* Kernel (d), fused form: the same GEMV with the activations given as f32
 * x [m, ldx] (ldx % 4 == 0, x 16-byte aligned) and quantised to Q8_K inside
 * the kernel, for 1..4 projections of one kind that share x (q/k/v, gate/up):
 * out[i][mi * ldo[i] + ni] for member i. Bit-identical to
 * rocknpu_hip_quantize_q8_k followed by rocknpu_hip_gemv_q8_k per member.
 * `w`, `w_bytes`, `n`, `out`, `ldo` are host arrays of `count` entries
 * (device pointers inside). */
int rocknpu_hip_gemv_q_f32(uint32_t kind, size_t count, const uint8_t * const * w,
                           const size_t * w_bytes, const size_t * n, size_t k, const float * x,
                           size_t ldx, size_t m, float * const * out, const size_t * ldo,
                           void * stream);

/* Bytes of the decode cache's tile-interleaved copy of a Q4_K (kind 4) or Q6_K
 * (kind 6) weight of n rows and K = k (a multiple of 256): whole 16-row tiles
 * of k/256 blocks each, ceil(n / 16) * 16 * (k / 256) * block bytes (the last
 * tile's missing rows are zero blocks). 0 for an invalid kind or shape. Host
 * code only. No counterpart in the reference, whose decode GEMV runs on the
 * CPU on ggml's row-major blocks. */
size_t rocknpu_hip_gemv_tiled_bytes(uint32_t kind, size_t k, size_t n);

/* Writes the tile-interleaved copy of the raw row-major GGUF blocks `w`
 * (w_bytes = n * k/256 * block bytes, 2-byte aligned) to `tiled` (16-byte
 * aligned, tiled_bytes >= rocknpu_hip_gemv_tiled_bytes): 16 rows' block b
 * together, each wave lane's operand bytes contiguous, so the decode GEMV
 * loads whole cache lines. The same bytes in another order (a one-time
 * conversion, like the W8 repack); the GEMV's results on the copy equal those
 * on the raw blocks bit for bit. No counterpart in the reference. */
int rocknpu_hip_gemv_tile_weights(uint32_t kind, const uint8_t * w, size_t w_bytes, size_t k, size_t n,
                                  uint8_t * tiled, size_t tiled_bytes, void * stream);

/* rocknpu_hip_gemv_q_f32 and rocknpu_hip_gemv_q8_k on tiled copies
 * (rocknpu_hip_gemv_tile_weights; w_bytes[i] = rocknpu_hip_gemv_tiled_bytes of
 * member i): the matrix-core GEMV with whole-line weight loads at every m
 * (launches of up to 16 rows for Q4_K, 8 for Q6_K). A row's f32 sum runs in the
 * order of the matrix-core kernel on raw blocks, so results equal
 * rocknpu_hip_gemv_q_f32 / _q8_k wherever that kernel serves the call, and
 * fused, grouped and Q8_K-input calls agree bit for bit.
 *
 * K split: launches of 2 to 8 rows over rows of 17 to 31 blocks (K 4352 to
 * 7936, e.g. a 5632-wide down projection; 2 ranges up to 4 rows, 4 from 5),
 * and of 1 to 8 rows over rows of 32 to 64 blocks (K 8192 to 16384; 4
 * ranges), split each 16-row tile's blocks into ranges on as many workgroups, whose partial sums meet in the workspace
 * (rocknpu_hip_gemv_tiled_workspace_bytes for the call's m, k and total rows;
 * 256-byte aligned; zeroed before its first use). Such a row's sum is the
 * ranges' sums added pairwise in a fixed tree, the same bits in grouped,
 * separate, fused and Q8_K-input calls, but not those of the unsplit kernels. Every completed call leaves the
 * workspace as it found it; calls that share one must not overlap (one per
 * stream). A call that finds it not clear sets its error word
 * (rocknpu_hip_gemv_tiled_workspace_check) and writes NaN, or the exact
 * value, where it did; never other bits. Calls that do not
 * split ignore workspace (it may be null); a split call without one large
 * enough returns ROCKNPU_STATUS_INVALID_ARGUMENT. No counterpart in the
 * reference. */
int rocknpu_hip_gemv_q_f32_tiled(uint32_t kind, size_t count, const uint8_t * const * w,
                                 const size_t * w_bytes, const size_t * n, size_t k, const float * x,
                                 size_t ldx, size_t m, float * const * out, const size_t * ldo,
                                 void * workspace, size_t workspace_bytes, void * stream);
int rocknpu_hip_gemv_q8_k_tiled(uint32_t kind, const uint8_t * w, size_t w_bytes, size_t k, size_t n,
                                const uint8_t * q8k, size_t m, float * out, size_t ldo, void * workspace,
                                size_t workspace_bytes, void * stream);

/* Bytes of the K-split workspace a tiled call of m activation rows over K = k
 * and `rows` output rows in all (the members' n summed) needs; 0 when none of
 * its launches splits. Host code only. No counterpart in the reference. */
size_t rocknpu_hip_gemv_tiled_workspace_bytes(uint32_t kind, size_t m, size_t k, size_t rows);

/* Waits for `stream`, then reads and clears the workspace's error word:
 * ROCKNPU_STATUS_OK when no split call on it found it not clear since the last
 * check, else ROCKNPU_STATUS_EXECUTION_ERROR, and the workspace must be zeroed
 * before it is used again. No counterpart in the reference. */
int rocknpu_hip_gemv_tiled_workspace_check(void * workspace, void * stream);

/* Whether a decode GEMV of m activation rows over Q4_K (kind 4) or Q6_K
 * (kind 6) rows of K = k runs faster on the tiled copy (1) or on the raw rows
 * (0): the tiled copy from two rows; at one row for rows of 5-16 blocks, of
 * 17-31 blocks that do not fill 8 block slots a row in whole passes (17-20 and
 * 25-27), and of 32 or more (Q6_K: up to 64); other one-row launches (rows of
 * at most 4 blocks, of 21-24 or 28-31, Q6_K rows beyond 64) keep the
 * lane-per-block and LDS-stream kernels on raw rows.
 * Host code only. No counterpart in the reference. */
int rocknpu_hip_gemv_tiled_preferred(uint32_t kind, size_t m, size_t k);

/* Stall report of rocknpu_hip_gemv_q_f32 and rocknpu_hip_gemv_q8_k. In the
 * fused lane-per-block kernel (rocknpu_hip_gemv_shape: *mfma == 0) and in the
 * Q6_K stream kernel (*mfma == 2, fused or not) a workgroup's waves wait for
 * the waves that stage the activations with a bounded poll (about 2^24
 * sleeps). A wave whose poll runs out writes NaN for each of its outputs and
 * sets a process-wide flag in pinned host memory. Call after synchronising
 * the streams of the launches to check: returns 1 if a launch gave up since
 * the last call, else 0, and clears the flag. The fused decode entry point of
 * the C ABI (rocknpu_matmul_q_q8k_group_f32_f32) checks it after its own
 * synchronisation and returns ROCKNPU_STATUS_EXECUTION_ERROR. The flag is
 * shared by every stream and thread of the process, and allocated by the
 * first launch with such a wait (a caller that captures launches into a HIP
 * graph makes one launch before capturing). No counterpart in the reference,
 * whose decode GEMV runs on the CPU. */
int rocknpu_hip_gemv_take_stall(void);

/* Test hook for the stall path: with spins > 0, later launches with the wait
 * above wait for one more arrival than exists and give up after `spins` polls
 * (every wave then exits normally, outputs NaN, flag set); spins == 0 restores
 * normal launches. Returns 0, or -1 for spins < 0. */
int rocknpu_hip_gemv_test_stall(int spins);

#ifdef __cplusplus
}
#endif

#endif

/*
 * breeze_qmm.h -- C ABI of the MI355X (gfx950) quantized linear library.
 *
 * The first block of entry points keeps the names, argument order and error
 * conventions of the reference CPU kernel's C ABI (kernel/quantized_matmul.cpp,
 * bound from Python by breeze/cpu_backend.py:15-54), so code written against
 * that ABI can load this library instead.  Host pointers in, host pointers
 * out, synchronous.
 *
 * The second block adds what a GPU caller needs: device-pointer entry points
 * on a caller's HIP stream (for PyTorch-ROCm tensors), an error string, the
 * fused LM-head argmax, and introspection hooks used by the parity tests.
 *
 * Threading: like the reference, settings are process-global and callers
 * serialize calls that share a device (the library keeps one activation
 * workspace per device).  A handle is bound to the device that was current
 * when it was packed.
 */
#ifndef BREEZE_QMM_H
#define BREEZE_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference ABI --------------------------------------------------- */

/* Replaces i4_set_threads (quantized_matmul.cpp:474).  Accepted and ignored:
 * the GPU path has no host thread pool. */
void i4_set_threads(int n);

/* Replaces i4_set_numa_split (quantized_matmul.cpp:475).  Accepted and
 * ignored: there is no NUMA weight replica on one GPU. */
void i4_set_numa_split(int cpu);

/* Replaces i4_set_hi_prec (quantized_matmul.cpp:476): 1 = two-pass INT16
 * activations, 0 = INT8 activations.  Process-global; default 0. */
void i4_set_hi_prec(int on);

/* Replaces i4_prepack_onnx (quantized_matmul.cpp:505-520).
 * qw: MatMulNBits bytes [N, K/32, 4*bits]; scales: [N, K/32] fp16
 * (scale_bits 16) or fp32 (32); qzeros: packed INT4 zero points
 * [N, ceil(K/64)] or NULL (INT8 must pass NULL).  Host pointers; the handle
 * owns device copies.  NULL on a contract violation (N<=0, K<=0, N%16, K%32,
 * bits not 4/8, scale_bits not 16/32, INT8 with qzeros) or on failure;
 * i4_last_error() says which. */
void* i4_prepack_onnx(const uint8_t* qw, const void* scales, const uint8_t* qzeros,
                      int N, int K, int bits, int scale_bits);

/* Replaces i4_prepack (quantized_matmul.cpp:480-499): the reference's
 * pre-transformed VNNI layout (B [N/16, nblk, 8, 32|64], scale/zp/corr
 * [N/16, nblk, 16]).  The supplied corr is honoured exactly as the reference
 * honours it, including values that differ from 128*sum(w - zp). */
void* i4_prepack(const uint8_t* B, const float* scale, const int8_t* zp,
                 const int32_t* corr, int N, int K, int nblk, int bits);

/* Replaces i4_free (quantized_matmul.cpp:522-524).  NULL is ignored. */
void i4_free(void* handle);

/* Replaces i4_matmul (quantized_matmul.cpp:528-552): C[M,N] = A[M,K] times
 * the packed weights, FP32, host pointers, blocking.  Like the reference it
 * returns nothing; on failure C is left unwritten and i4_last_error() is set
 * (the Python bridge turns that into RuntimeError). */
void i4_matmul(void* handle, const float* A, int M, float* C);

/* Replaces i4_matmul_region (quantized_matmul.cpp:558-572).  There is no
 * OpenMP region on the GPU path: this is i4_matmul, and the caller's scratch
 * and ascale buffers are not used. */
void i4_matmul_region(void* handle, const float* A, int M, float* C,
                      uint8_t* scratch, float* ascale);

/* ---- GPU additions (no counterpart in the reference) ----------------- */

/* Message for the last failure on this thread ("" if none). */
const char* i4_last_error(void);

/* 1 if a usable gfx950 device and this library's kernels are present. */
int i4_device_ok(void);

/* i4_matmul on device pointers, asynchronous on `stream` (a hipStream_t, or
 * NULL for the null stream).  dA: fp32 [M,K], dC: fp32 [M,N], both 16-byte
 * aligned.  Returns 0, or a negative code with i4_last_error() set. */
int i4_matmul_dev(void* handle, const float* dA, int M, float* dC, void* stream);

/* As i4_matmul_dev, and also writes, for each row m, the index of the first
 * maximum of C[m,:] (NaN counts as the maximum, -0 equals +0; numpy.argmax
 * semantics) to dIdx[m] (int64).  Used for the LM head. */
int i4_matmul_argmax_dev(void* handle, const float* dA, int M, float* dC,
                         int64_t* dIdx, void* stream);

/* Fused gate/up projection of a decoder MLP, replacing the two i4_matmul calls
 * and the SiLU loop of kernel/qwen35_decoder.cpp:406-408:
 *   dC[M,N] = silu(dA * Wgate) * (dA * Wup),  silu(x) = x / (1 + exp(-x)).
 * Both projections are bit-identical to i4_matmul_dev's, and the SiLU and
 * product are the reference's bit for bit (its expf, the host C library's,
 * restated on the device).  When a decode launch takes both projections it
 * is one launch (SiLU and product in the epilogue); otherwise two launches
 * and i4_silu_mul_dev's kernel.  Returns as i4_matmul_dev. */
int i4_matmul_silu_mul_dev(void* gate, void* up, const float* dA, int M, float* dC, void* stream);

/* The decoder MLP's elementwise step on device pointers, replacing the loop
 * g1[i] = siluf(g1[i]) * g2[i] of kernel/qwen35_decoder.cpp:408 (siluf at
 * 128): dOut[i] = dG[i] / (1 + expf(-dG[i])) * dU[i] for i < n, bit for bit
 * the reference's (its expf is the host C library's; the device restates
 * it).  dOut may equal dG or dU.  Asynchronous on `stream`.  Returns 0, or a
 * negative code with i4_last_error() set. */
int i4_silu_mul_dev(const float* dG, const float* dU, size_t n, float* dOut, void* stream);

/* i4_matmul_dev, or i4_matmul_argmax_dev when dIdx is not NULL, that
 * allocates nothing: no hipMalloc, hipFree or allocating library call.  It
 * has no counterpart in the reference; it is for callers that cannot
 * allocate, such as code under HIP graph capture or serving loops that
 * forbid it.  All of its device scratch is one static 16 MiB array per
 * device, so a call whose activation records do not fit is refused (-4,
 * i4_last_error() says why): 72 bytes per row and 32-block of K when
 * the decode kernel stages its records (up to 32 rows, M*K above 16384), with
 * K counted rounded up to a multiple of 128 and, from 5 to 32 rows, M rounded
 * up to a multiple of 8 (the eight-row groups' records cover whole groups), and
 * about 68 bytes per 32-block of K per row, rows rounded up to 32, 64 or 128, for
 * the rows the prefill GEMM takes; a split-K call (few column tiles over a long
 * K) takes 4 bytes per 16-column tile rounded up to 256, plus 68 bytes per row
 * and 32-block of K (K rounded up to a multiple of 128) per tile.  Calls that
 * overlap on one device share the array and race: serialize them.  Outputs are those of i4_matmul_dev /
 * i4_matmul_argmax_dev, bit for bit. */
int i4_matmul_noalloc_dev(void* handle, const float* dA, int M, float* dC, int64_t* dIdx, void* stream);

/* Several projections of one activation in one launch, replacing
 * consecutive i4_matmul calls on the same input (kernel/qwen35_decoder.cpp:
 * 285-288 in_qkv, in_z, in_b, in_a; 334-336 q, k, v):
 *   dC[i][M, N_i] = dA[M, K] * W_i,  i < n <= 4, one K for all.
 * Each output is bit-identical to i4_matmul_dev's.  With M <= 8 and handles
 * of one device layout (all but N alike, no per-block metadata) it is one
 * decode launch whose workgroups share out the concatenated column tiles
 * (the activation is quantized once per workgroup, and small projections
 * ride along with large ones); otherwise one launch per handle.  Returns as
 * i4_matmul_dev. */
int i4_matmul_multi_dev(void* const* handles, int n, const float* dA, int M, float* const* dC, void* stream);

/* The decoder's RMSNorm followed by the projections of its output, replacing
 * rmsnorm(hn, h, w) and the i4_matmul calls on hn that follow it
 * (kernel/qwen35_decoder.cpp:279 and 285-288, 405-407, 419-420):
 *   hn = rmsnorm(dX[M, K], dNormW[K], eps),  dC[i][M, N_i] = hn * W_i.
 * hn is bit-identical to i4_rmsnorm_dev's and every output to
 * i4_matmul_dev's on it.  When the decode kernel quantizes the activation
 * itself (M <= 8 with M <= 4 rows of K/32 <= 512/M blocks, e.g. up to three
 * rows of K = 5120) and the handles share a device layout, the norm runs in
 * the prologue of the one projection launch; otherwise it is its own launch
 * first.  dHn (may be NULL) receives hn [M, K].  Returns as i4_matmul_dev. */
int i4_rmsnorm_matmul_multi_dev(const float* dX, const float* dNormW, float eps, void* const* handles, int n, int M,
                                float* const* dC, float* dHn, void* stream);

/* Routing introspection, for tests: the plan the library makes for a call
 * of M rows on a handle of N columns, K and `bits`, without a device or a
 * handle.  flags: 1 block-integer export, 2 argmax, 4 gate/up pair,
 * 8 multi-projection (one segment of N), 16 RMSNorm in that launch,
 * 32 per-block metadata (explicit zero points or small scale groups),
 * 64 legacy corr; n_cu: compute units of the device.  out[0..16] = route
 * (1 decode in four-row groups, 2 decode in eight-row groups, 3 prefill
 * GEMM, 4 rows kernel, 0 no single launch takes a paired or multi call),
 * stand-alone quantizer (0 none: the decode prologue quantizes, 1 staged
 * records, 2 eight-row records, 3 prefill records), prologue quantizes,
 * block pairs, records in LDS, rows per row group, row groups, tile ranges,
 * row groups of a tile range on one XCD, LDS bytes, prefill row pairs,
 * prefill column tiles, grid x, grid y, split-K workgroups per tile (0:
 * none), non-temporal weight loads, phases across tile boundaries.
 * Environment overrides apply as for
 * a call.  Returns the number of values written (at most nout), or -1. */
int i4_plan_query(int bits, int M, int K, int N, int flags, int n_cu, int32_t* out, int nout);

/* Handle facts: out[0..7] = N, K, bits, scale group (blocks per distinct
 * scale, 0 = one per column), has_zero_points, has_corr_delta,
 * device bytes held, device ordinal.  Returns 0 or -1. */
int i4_handle_info(void* handle, int64_t* out);

/* Reads a handle back into MatMulNBits form on the host: qw [N, K/32,
 * 4*bits] bytes, scales fp32 [N, K/32], zp [N, K/32] (one byte per block,
 * the zero point actually applied) and corr_delta int32 [N, K/32]
 * (128*sum(w - zp) - corr, zero unless a legacy corr disagreed).  Any output
 * pointer may be NULL.  Lets tests pin the packed layout semantically. */
int i4_unpack(void* handle, uint8_t* qw, float* scales, uint8_t* zp, int32_t* corr_delta);

/* Debug export of the exact per-(row, column, 32-block) integer dot products
 * cs = sum_k q[m,k] * b[n,k] (plus the legacy corr term) that feed the FP32
 * epilogue: dCs int32 [M, N, K/32].  Same kernels as i4_matmul_dev. */
int i4_block_dots_dev(void* handle, const float* dA, int M, int32_t* dCs, void* stream);

/* The decoder's RMSNorm (kernel/qwen35_decoder.cpp:134-140, an internal
 * function there, called ahead of the projections at 279, 405 and 420) on
 * device pointers: dOut[m, :] = (dX[m, :] * inv) * dW with
 * inv = 1 / sqrtf((float)(ss / H) + eps) and ss the double sum of squares
 * in element order, bit-identical to the reference's.  Asynchronous on
 * `stream`.  Returns 0, or a negative code with i4_last_error() set. */
int i4_rmsnorm_dev(const float* dX, const float* dW, int M, int H, float eps, float* dOut, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BREEZE_QMM_H */

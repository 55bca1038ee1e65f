/*
 * qmm_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Scalar CPU restatement of Breeze's quantized linear path: MatMulNBits
 * INT4/INT8 weights (block size 32) times activations quantized per
 * (row, 32-block) to INT16 (two-pass, "hi_prec") or INT8, FP32 output.
 * Only the tests, the smoke check and the benchmark's CPU leg may load it,
 * and only as the checker; the product library never links it.
 *
 * Every function cites the reference lines it restates (paths are relative
 * to the breeze-engine repository):
 *   kernel/quantized_matmul.cpp   packing, activation quantizers, tile kernels
 *   breeze/quant.py               MatMulNBits dequant contract (zero points)
 *   breeze/cpu_backend.py         prepack validation and the legacy layout
 *   kernel/qwen35_decoder.cpp     the decoder's RMSNorm ahead of the projections
 *
 * Build: see oracle/Makefile (-ffp-contract=off, no fast-math), so each
 * float operation below rounds exactly once, as written.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

ORC_API int orc_version(void) { return 1; }

/* FP16 bits -> FP32, exact for normals, subnormals, signed zeros and
 * infinities; NaNs come out quiet with their payload kept, as F16C
 * VCVTPH2PS does (quantized_matmul.cpp:157, _cvtsh_ss). */
ORC_API float orc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int shift = 0;
            while (!(man & 0x400u)) { man <<= 1; ++shift; }
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(113 - shift) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* One (row, 32-block) of activation quantization.
 * quantize_A_i16 (quantized_matmul.cpp:237-258) with qmax=32767 and
 * quantize_A (215-232) with qmax=127:
 *   amax = max |a| by `v > amax` from +0 (so NaNs are skipped),
 *   s = amax / qmax, inv = s > 0 ? 1/s : 0, q = clamp(lrint(a*inv), +-qmax).
 * A non-finite product a*inv gives q = 0: the reference's (int)lrint() lowers
 * to the 64-bit cvtss2si, whose "integer indefinite" LONG_MIN truncates to 0.
 * Also returns sum(q), which the GPU path uses for zero-point corrections. */
static void quant_block(const float* a, int qmax, int16_t* q, float* sa, int32_t* sq) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        float v = fabsf(a[i]);
        if (v > amax) amax = v;
    }
    float s = amax / (float)qmax;
    float inv = s > 0.0f ? 1.0f / s : 0.0f;
    int32_t sum = 0;
    for (int i = 0; i < 32; ++i) {
        float p = a[i] * inv;
        int v = isfinite(p) ? (int)lrintf(p) : 0;
        v = v > qmax ? qmax : (v < -qmax ? -qmax : v);
        q[i] = (int16_t)v;
        sum += v;
    }
    *sa = s;
    *sq = sum;
}

/* A fp32 [M,K] -> q int16 [M,K], sa fp32 [M,K/32], sq int32 [M,K/32]
 * (sq may be NULL).  hi_prec selects INT16 (quantize_A_i16) or INT8
 * (quantize_A) as i4_matmul does (quantized_matmul.cpp:531-536). */
ORC_API void orc_quantize(const float* A, int M, int K, int hi_prec,
                          int16_t* q, float* sa, int32_t* sq) {
    const int nblk = K / 32, qmax = hi_prec ? 32767 : 127;
    for (int m = 0; m < M; ++m)
        for (int j = 0; j < nblk; ++j) {
            int32_t s;
            quant_block(A + (size_t)m * K + 32 * j, qmax, q + (size_t)m * K + 32 * j,
                        sa + (size_t)m * nblk + j, &s);
            if (sq) sq[(size_t)m * nblk + j] = s;
        }
}

/* The two unsigned byte halves the reference feeds VPDPBUSD in INT16 mode:
 * u = q + 32768, hi = u >> 8, lo = u & 255 (quantized_matmul.cpp:252-254). */
ORC_API void orc_split_hilo(const int16_t* q, size_t n, uint8_t* hi, uint8_t* lo) {
    for (size_t i = 0; i < n; ++i) {
        unsigned u = (unsigned)((int)q[i] + 32768);
        hi[i] = (uint8_t)(u >> 8);
        lo[i] = (uint8_t)(u & 0xFFu);
    }
}

/* MatMulNBits -> signed weights b [N,K] (int16) and fp32 scales [N,K/32].
 *   4-bit: byte i of a block holds k=2i (low nibble) and k=2i+1 (high),
 *          b = nibble - zp, zp from packed qzeros (low nibble = even block)
 *          or 8 (quant.py:40-54; quantized_matmul.cpp:182), int8 wraparound
 *          as _mm512_sub_epi8 (quantized_matmul.cpp:299).
 *   8-bit: b = byte - 128, zp fixed at 128 (quant.py:33; cpp:172).
 *   scales: fp16 (scale_bits 16) or fp32 (32) per (column, block)
 *          (quantized_matmul.cpp:156-159).
 * Returns 0, or -1 on a contract violation (quantized_matmul.cpp:66-67,
 * 507-508). */
ORC_API int orc_unpack_nbits(const uint8_t* qw, const void* scales, const uint8_t* qzeros,
                             int N, int K, int bits, int scale_bits,
                             int16_t* b, float* sb) {
    if (!qw || !scales || N <= 0 || K <= 0 || N % 16 || K % 32 ||
        (bits != 4 && bits != 8) || (scale_bits != 16 && scale_bits != 32) ||
        (bits == 8 && qzeros))
        return -1;
    const int nblk = K / 32, bb = 4 * bits;
    for (int n = 0; n < N; ++n)
        for (int j = 0; j < nblk; ++j) {
            const size_t blk = (size_t)n * nblk + j;
            const uint8_t* src = qw + blk * bb;
            int16_t* dst = b + (size_t)n * K + 32 * j;
            if (scale_bits == 16)
                sb[blk] = orc_half_to_float(((const uint16_t*)scales)[blk]);
            else
                sb[blk] = ((const float*)scales)[blk];
            if (bits == 8) {
                for (int i = 0; i < 32; ++i) dst[i] = (int16_t)((int)src[i] - 128);
            } else {
                int zp = qzeros ? (qzeros[(size_t)n * ((nblk + 1) / 2) + j / 2] >> (4 * (j % 2))) & 15 : 8;
                for (int i = 0; i < 16; ++i) {
                    dst[2 * i] = (int16_t)(int8_t)(uint8_t)((src[i] & 15) - zp);
                    dst[2 * i + 1] = (int16_t)(int8_t)(uint8_t)((src[i] >> 4) - zp);
                }
            }
        }
    return 0;
}

/* Legacy pre-transformed layout (i4_prepack, quantized_matmul.cpp:480-499):
 *   B int4 [N/16, nblk, 8, 32]: per k-group g of 4, 64 nibbles v[col*4+k]
 *          stored low-nibble-first (unpack_kgroup, 204-213); b = v - zp
 *          with int8 wraparound (299).
 *   B int8 [N/16, nblk, 8, 64]: signed bytes v[col*4+k] (320-365).
 *   scale, zp, corr [N/16, nblk, 16].
 * Outputs b [N,K], sb [N,nblk] and delta [N,nblk] = 128*sum_k(b) - corr,
 * the amount by which the supplied corr departs from the one pack_onnx
 * would compute (quantized_matmul.cpp:190).  hp_combine (262-268) then gives
 * cs = sum(q*b) + 256*delta in INT16 mode and sum(q*b) + delta in INT8 mode. */
ORC_API int orc_unpack_legacy(const uint8_t* B, const float* scale, const int8_t* zp,
                              const int32_t* corr, int N, int K, int nblk, int bits,
                              int16_t* b, float* sb, int32_t* delta) {
    if (!B || !scale || !corr || (bits == 4 && !zp) || N <= 0 || K <= 0 || N % 16 ||
        K % 32 || nblk != K / 32 || (bits != 4 && bits != 8))
        return -1;
    const int ntiles = N / 16, gbytes = bits == 8 ? 64 : 32;
    for (int t = 0; t < ntiles; ++t)
        for (int j = 0; j < nblk; ++j) {
            const size_t meta = ((size_t)t * nblk + j) * 16;
            const uint8_t* blk = B + ((size_t)t * nblk + j) * 8 * gbytes;
            for (int col = 0; col < 16; ++col) {
                const int n = t * 16 + col;
                int16_t* dst = b + (size_t)n * K + 32 * j;
                int32_t sum = 0;
                for (int g = 0; g < 8; ++g)
                    for (int k = 0; k < 4; ++k) {
                        const int v = col * 4 + k;
                        int val;
                        if (bits == 8) {
                            val = (int8_t)blk[g * 64 + v];
                        } else {
                            const uint8_t byte = blk[g * 32 + v / 2];
                            const int nib = (v & 1) ? byte >> 4 : byte & 15;
                            val = (int8_t)(uint8_t)(nib - zp[meta + col]);
                        }
                        dst[g * 4 + k] = (int16_t)val;
                        sum += val;
                    }
                sb[(size_t)n * nblk + j] = scale[meta + col];
                delta[(size_t)n * nblk + j] = 128 * sum - corr[meta + col];
            }
        }
    return 0;
}

/* cs[m,n,j] = sum_k q[m,k] * b[n,k] over block j, exact.  This is the value
 * hp_combine reconstructs from the two VPDPBUSD passes:
 * ((acc_hi - corr) << 8) + acc_lo == sum(q*b) when corr = 128*sum(b)
 * (quantized_matmul.cpp:260-268, 303-312, 350-359).  |cs| < 2^27. */
ORC_API void orc_block_dots(const int16_t* q, int M, const int16_t* b, int N, int K,
                            int32_t* cs) {
    const int nblk = K / 32;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < nblk; ++j) {
                const int16_t* x = q + (size_t)m * K + 32 * j;
                const int16_t* w = b + (size_t)n * K + 32 * j;
                int64_t s = 0;
                for (int i = 0; i < 32; ++i) s += (int64_t)x[i] * w[i];
                cs[((size_t)m * N + n) * nblk + j] = (int32_t)s;
            }
}

/* The FP32 epilogue, per output (m, n), blocks in ascending order from +0:
 *   acc = fmaf(sa[m,j], (float)cs[m,n,j] * sb[n,j], acc)
 * (_mm512_cvtepi32_ps, _mm512_mul_ps, _mm512_fmadd_ps at
 * quantized_matmul.cpp:311-315 and 358-362; store at 317/364). */
ORC_API void orc_chain(const int32_t* cs, const float* sa, const float* sb, int M, int N,
                       int nblk, float* C) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.0f;
            const int32_t* c = cs + ((size_t)m * N + n) * nblk;
            for (int j = 0; j < nblk; ++j) {
                float f = (float)c[j] * sb[(size_t)n * nblk + j];
                acc = fmaf(sa[(size_t)m * nblk + j], f, acc);
            }
            C[(size_t)m * N + n] = acc;
        }
}

/* Shared tail of the two full-path entry points below. */
static int run_path(const int16_t* b, const float* sb, const int32_t* delta, int N, int K,
                    const float* A, int M, int hi_prec, float* C, int32_t* cs_out) {
    const int nblk = K / 32;
    const int32_t mult = hi_prec ? 256 : 1;
    int16_t* q = malloc(sizeof(int16_t) * (size_t)M * K);
    float* sa = malloc(sizeof(float) * (size_t)M * nblk);
    int rc = -2;
    if (q && sa) {
        orc_quantize(A, M, K, hi_prec, q, sa, NULL);
        if (cs_out) {
            orc_block_dots(q, M, b, N, K, cs_out);
            if (delta)
                for (int m = 0; m < M; ++m)
                    for (int n = 0; n < N; ++n)
                        for (int j = 0; j < nblk; ++j)
                            cs_out[((size_t)m * N + n) * nblk + j] += mult * delta[(size_t)n * nblk + j];
            orc_chain(cs_out, sa, sb, M, N, nblk, C);
        } else {
            /* The same block integers and chain as orc_block_dots,
             * the delta term and orc_chain, one output at a time (outputs
             * are independent, so the threads change no bit). */
#pragma omp parallel for schedule(static)
            for (long long mn = 0; mn < (long long)M * N; ++mn) {
                const int m = (int)(mn / N), n = (int)(mn % N);
                float acc = 0.0f;
                for (int j = 0; j < nblk; ++j) {
                    const int16_t* x = q + (size_t)m * K + 32 * j;
                    const int16_t* w = b + (size_t)n * K + 32 * j;
                    int64_t s = 0;
                    for (int i = 0; i < 32; ++i) s += (int64_t)x[i] * w[i];
                    int32_t c = (int32_t)s;
                    if (delta) c += mult * delta[(size_t)n * nblk + j];
                    const float f = (float)c * sb[(size_t)n * nblk + j];
                    acc = fmaf(sa[(size_t)m * nblk + j], f, acc);
                }
                C[mn] = acc;
            }
        }
        rc = 0;
    }
    free(q);
    free(sa);
    return rc;
}

/* i4_prepack_onnx + i4_matmul (quantized_matmul.cpp:505-552) in one call:
 * C [M,N] from MatMulNBits weights and fp32 A [M,K].  Rows are independent,
 * so the reference's 8-row chunking (542-550) does not change any value.
 * cs_out, if not NULL, receives the [M,N,K/32] block integers. */
ORC_API int orc_matmul_nbits(const uint8_t* qw, const void* scales, const uint8_t* qzeros,
                             int N, int K, int bits, int scale_bits, const float* A, int M,
                             int hi_prec, float* C, int32_t* cs_out) {
    if (M < 0) return -1;
    int16_t* b = malloc(sizeof(int16_t) * (size_t)N * K);
    float* sb = malloc(sizeof(float) * (size_t)N * (K / 32));
    int rc = -2;
    if (b && sb) {
        rc = orc_unpack_nbits(qw, scales, qzeros, N, K, bits, scale_bits, b, sb);
        if (rc == 0) rc = run_path(b, sb, NULL, N, K, A, M, hi_prec, C, cs_out);
    }
    free(b);
    free(sb);
    return rc;
}

/* i4_prepack (legacy layout) + i4_matmul. */
ORC_API int orc_matmul_legacy(const uint8_t* B, const float* scale, const int8_t* zp,
                              const int32_t* corr, int N, int K, int nblk, int bits,
                              const float* A, int M, int hi_prec, float* C) {
    if (M < 0) return -1;
    int16_t* b = malloc(sizeof(int16_t) * (size_t)N * K);
    float* sb = malloc(sizeof(float) * (size_t)N * (K / 32));
    int32_t* delta = malloc(sizeof(int32_t) * (size_t)N * (K / 32));
    int rc = -2;
    if (b && sb && delta) {
        rc = orc_unpack_legacy(B, scale, zp, corr, N, K, nblk, bits, b, sb, delta);
        if (rc == 0) rc = run_path(b, sb, delta, N, K, A, M, hi_prec, C, NULL);
    }
    free(b);
    free(sb);
    free(delta);
    return rc;
}

/* RMSNorm of the decoder (qwen35_decoder.cpp:134-140): per row, the sum of
 * squares is accumulated in double, one element after the other from j = 0;
 * inv = 1 / sqrtf((float)(ss / H) + eps) in float (correctly rounded divide
 * and square root); out = (x * inv) * w, two float roundings. */
ORC_API void orc_rmsnorm(const float* x, const float* w, int s, int H, float eps, float* out) {
    for (int i = 0; i < s; ++i) {
        const float* xr = x + (size_t)i * H;
        float* o = out + (size_t)i * H;
        double ss = 0;
        for (int j = 0; j < H; ++j) ss += (double)xr[j] * xr[j];
        const float inv = 1.0f / sqrtf((float)(ss / H) + eps);
        for (int j = 0; j < H; ++j) o[j] = xr[j] * inv * w[j];
    }
}

/* The double sum of squares alone (the first line of the row loop above),
 * for tests of the sum's exactness. */
ORC_API void orc_sumsq(const float* x, int s, int H, double* ss_out) {
    for (int i = 0; i < s; ++i) {
        const float* xr = x + (size_t)i * H;
        double ss = 0;
        for (int j = 0; j < H; ++j) ss += (double)xr[j] * xr[j];
        ss_out[i] = ss;
    }
}

/* The decoder MLP's elementwise step (qwen35_decoder.cpp:408, siluf at 128):
 * out[i] = g[i] / (1 + expf(-g[i])) * u[i] in float, where expf is the host
 * C library's, the very function the reference's std::exp(float) calls.
 * Rows are independent, so the loop is split over OpenMP threads. */
ORC_API void orc_silu_mul(const float* g, const float* u, long long n, float* out) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; ++i) out[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

// qmm.hip -- MI355X (gfx950) quantized linear path: MatMulNBits INT4/INT8
// weights x per-(row, 32-block) quantized activations, FP32 out.
//
// Arithmetic contract (kernel/quantized_matmul.cpp of breeze-engine):
//   activations, per row m and block j of 32 k (quantize_A_i16 237-258 /
//   quantize_A 215-232): amax = max|a| (NaN skipped), s = amax/qmax,
//   inv = s>0 ? 1/s : 0, q = clamp(rint(a*inv), +-qmax), qmax 32767 or 127;
//   a non-finite a*inv gives q = 0 (the reference's (int)lrint).
//   block integer cs = sum_k q*b, b = nibble - zp (INT4) or byte - 128 (INT8)
//   (pack_onnx 140-194, hp_combine 262-268);
//   C[m,n] = fold over j ascending of acc = fma(s[m,j], f32(cs)*scale[n,j],
//   acc) from +0 (tile_kernel 311-315 / tile_kernel8 358-362).
//
// gfx950 realisation:
//   * INT16 activations are split into two SIGNED bytes, h = (u>>8)-128 and
//     l = (u&255)-128 with u = q+32768, so q = 256h + l + 128 and
//     cs = 256*H + L + 128*S with H = sum h*b, L = sum l*b, S = sum b.
//   * One v_mfma_i32_16x16x32_i8 covers exactly one 32-block for 16 weight
//     columns.  Its 16 A rows are four groups of [h row, l row, ones row,
//     zero row], one group per activation row, so H, L and S of an output
//     (m, n) land in registers 0..2 of the same lane and combine in-lane.
//   * INT4 weights stay raw nibbles 0..15 (valid signed bytes); the zero
//     point is applied as cs -= zp * sum(q), with sum(q) per (m, j) from the
//     quantizer.  INT8 weights are stored as signed bytes (raw ^ 0x80).
//   * The FP32 chain is evaluated in block order per (m, n), exactly as the
//     reference does, so outputs are bit-identical for every M and row m of
//     an M-row call equals a 1-row call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/breeze_qmm.h"
#include "qmm_common.h"

using namespace bq;

namespace {

// ------------------------------------------------------------------ errors

thread_local std::string g_err;
int g_hi_prec = 0;

void set_err(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
}

bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    set_err("%s: %s", what, hipGetErrorString(e));
    return false;
}

Handle* as_handle(void* p) {
    auto* h = static_cast<Handle*>(p);
    if (!h || h->magic != kMagic) {
        set_err("invalid handle");
        return nullptr;
    }
    return h;
}

// ------------------------------------------------------------------ repack

// MatMulNBits bytes (or signed bytes, raw_signed) -> device chunk layout.
__global__ void repack_kernel(const uint8_t* __restrict__ raw, uint4* __restrict__ out, int N,
                              int nblk, int nbg, int bits, int raw_signed) {
    const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)(N / 16) * nbg * 64;
    if (o >= total) return;
    const int lane = (int)(o & 63);
    const size_t tc = o >> 6;
    const int cg = (int)(tc % nbg);
    const int t = (int)(tc / nbg);
    const int n = t * 16 + (lane & 15), oct = lane >> 4;
    uint32_t w[4] = {0, 0, 0, 0};
    if (bits == 8) {
        const uint32_t x = raw_signed ? 0u : 0x80808080u;
        for (int hb = 0; hb < 2; ++hb) {
            const int j = cg * 2 + hb;
            if (j >= nblk) continue;
            const uint8_t* src = raw + ((size_t)n * nblk + j) * 32 + oct * 8;
            uint32_t lo = 0, hi = 0;
            for (int p = 0; p < 4; ++p) lo |= (uint32_t)src[p] << (8 * p);
            for (int p = 0; p < 4; ++p) hi |= (uint32_t)src[4 + p] << (8 * p);
            w[2 * hb] = lo ^ x;
            w[2 * hb + 1] = hi ^ x;
        }
    } else {
        for (int q = 0; q < 4; ++q) {
            const int j = cg * 4 + q;
            if (j >= nblk) continue;
            const uint8_t* src = raw + ((size_t)n * nblk + j) * 16 + oct * 4;
            uint32_t x = 0;
            for (int b = 0; b < 4; ++b) {
                const uint32_t lo = (src[b >> 1] >> (4 * (b & 1))) & 15u;
                const uint32_t hi = (src[2 + (b >> 1)] >> (4 * (b & 1))) & 15u;
                x |= (lo | hi << 4) << (8 * b);
            }
            w[q] = x;
        }
    }
    out[o] = make_uint4(w[0], w[1], w[2], w[3]);
}

// ------------------------------------------------------------------ quantize

// Stand-alone activation quantizer: 4 lanes per (row, block), 8 k each
// (quant4x8).  Records go
// to Aq [M][nblk][64 B]; scale and sum(q) to Sa/Sq [M][nblk4].
template <bool HP>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ A, int M, int K,
                                                       int nblk, int nblk4, uint8_t* __restrict__ Aq,
                                                       float* __restrict__ Sa, int* __restrict__ Sq) {
    const int gtid = blockIdx.x * 256 + threadIdx.x;
    const int blk = gtid >> 2, e = gtid & 3;
    const bool valid = blk < M * nblk;
    const int m = valid ? blk / nblk : 0, j = valid ? blk - m * nblk : 0;
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (valid) {
        const float* x = A + (size_t)m * K + 32 * j + 8 * e;
        v0 = *reinterpret_cast<const float4*>(x);
        v1 = *reinterpret_cast<const float4*>(x + 4);
    }
    float s;
    int sum;
    uint2 ph, pl;
    quant4x8<HP>(v0, v1, s, ph, pl, sum);
    if (valid) {
        uint8_t* rec = Aq + ((size_t)m * nblk + j) * 64;
        *reinterpret_cast<uint2*>(rec + 8 * e) = ph;
        *reinterpret_cast<uint2*>(rec + 32 + 8 * e) = pl;
        if (e == 0) {
            Sa[(size_t)m * nblk4 + j] = s;
            Sq[(size_t)m * nblk4 + j] = sum;
        }
    }
}

// The same quantizer for the decode kernel in row groups of eight
// (dec8_kernel): records in its MFMA A-operand order, per row group
// [chunk][JG / 2][64 lanes][16 B], lane 16 e + 2 m + s holding k-octet e of
// record part s of the group's row m for blocks 2 h and 2 h + 1 of the chunk
// (8 bytes each).  Rows past M (to the end of the last group) and the padding
// blocks of the last chunk are zeros.  Scales and sums of q as
// quantize_kernel's.  Threads: 8 rg_count rows x nblk_pad blocks x 4.
template <bool HP, int JG>
__global__ __launch_bounds__(256) void quantize_r8_kernel(const float* __restrict__ A, int M, int K, int nblk,
                                                          int nblk_pad, int nblk4, int rows, uint8_t* __restrict__ R,
                                                          float* __restrict__ Sa, int* __restrict__ Sq) {
    const int gtid = blockIdx.x * 256 + threadIdx.x;
    const int blk = gtid >> 2, e = gtid & 3;
    const bool in = blk < rows * nblk_pad;
    const int m = in ? blk / nblk_pad : 0, j = in ? blk - m * nblk_pad : 0;
    const bool real = in && m < M && j < nblk;
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (real) {
        const float* x = A + (size_t)m * K + 32 * j + 8 * e;
        v0 = *reinterpret_cast<const float4*>(x);
        v1 = *reinterpret_cast<const float4*>(x + 4);
    }
    float s;
    int sum;
    uint2 ph, pl;
    quant4x8<HP>(v0, v1, s, ph, pl, sum);
    if (in) {
        if (!real) ph = pl = make_uint2(0u, 0u);
        const int c = j / JG, jb = j - c * JG, ml = m & 7;
        uint8_t* base = R + (size_t)(m >> 3) * nblk_pad * 512 +
                        ((size_t)(c * (JG / 2) + (jb >> 1)) * 64) * 16 + (jb & 1) * 8;
        *reinterpret_cast<uint2*>(base + (16 * e + 2 * ml) * 16) = ph;
        *reinterpret_cast<uint2*>(base + (16 * e + 2 * ml + 1) * 16) = pl;
        if (real && e == 0) {
            Sa[(size_t)m * nblk4 + j] = s;
            Sq[(size_t)m * nblk4 + j] = sum;
        }
    }
}

// 128 * sum of the signed INT8 weights of each (column, block), tile-major
// per chunk ([N/16][nbg][16][2]): the bias term of the two-pass product,
// cs = 256*H + L + 128*S.  One thread per (tile, chunk, column).
__global__ __launch_bounds__(256) void wsum_kernel(const uint4* __restrict__ W, int32_t* __restrict__ WS,
                                                   int ntiles, int nbg) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)ntiles * nbg * 16) return;
    const int col = (int)(i & 15);
    const size_t tc = i >> 4;
    auto sum4 = [](uint32_t x) {
        return (int)(int8_t)x + (int)(int8_t)(x >> 8) + (int)(int8_t)(x >> 16) + (int)(int8_t)(x >> 24);
    };
    int s0 = 0, s1 = 0;
    for (int oct = 0; oct < 4; ++oct) {
        const uint4 w = W[tc * 64 + oct * 16 + col];
        s0 += sum4(w.x) + sum4(w.y);
        s1 += sum4(w.z) + sum4(w.w);
    }
    WS[i * 2] = 128 * s0;
    WS[i * 2 + 1] = 128 * s1;
}

// ------------------------------------------------------------------ generic rows kernel (legacy corr past the decode rows, block-integer export)
//
// One workgroup per (16-column tile, 8-row chunk), all of K: waves compute a
// segment of f values into LDS, then one lane per (m, n) folds them in order.

constexpr int kRowWaves = 4;
constexpr int kRowChunks = 2;
constexpr int kRowsPerWG = 8;

template <int BITS, bool HP, bool DOTS>
__global__ __launch_bounds__(kRowWaves * 64) void rows_kernel(GemvArgs a) {
    constexpr int JG = BITS == 8 ? 2 : 4;
    constexpr int SEG = kRowWaves * kRowChunks * JG;
    __shared__ float fbuf[kRowsPerWG][SEG][16];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x;
    const int m0 = blockIdx.y * kRowsPerWG;
    const int Mc = min(kRowsPerWG, a.M - m0);
    const int nmf = (Mc + 3) >> 2;
    const int col = lane & 15, grp = lane >> 4;
    const int arow = lane & 15, arg = arow >> 2, ars = arow & 3;
    const size_t n = (size_t)t * 16 + col;
    const int cm = threadIdx.x >> 4, ccol = threadIdx.x & 15;
    float acc = 0.0f;
    const uint2* Aq2 = reinterpret_cast<const uint2*>(a.Aq);

    const int nseg = (a.nblk + SEG - 1) / SEG;
    for (int s = 0; s < nseg; ++s) {
        const int j0 = s * SEG;
#pragma unroll
        for (int cc = 0; cc < kRowChunks; ++cc) {
            const int cg = j0 / JG + wave * kRowChunks + cc;
            if (cg * JG >= a.nblk) break;
            const uint4 wv = a.W[((size_t)t * a.nbg + cg) * 64 + lane];
#pragma unroll
            for (int jb = 0; jb < JG; ++jb) {
                const int j = cg * JG + jb;
                if (j >= a.nblk) break;
                const uint64_t bop = unpack_b(wv, jb, BITS);
                const int JGh = BITS == 8 ? 2 : 4;
                const float sc = (a.flags & kFlagScBlk) ? a.S[blk_index((int)n, j, a.nbg, JGh)]
                                                        : a.S[grp_index((int)n, j, a.ngrp, a.sc_shift)];
                for (int mi = 0; mi < nmf; ++mi) {
                    const int ml = mi * 4 + arg;
                    uint64_t aop = 0;
                    if (ars == 2) {
                        aop = 0x0101010101010101ull;
                    } else if (ars < 2 && ml < Mc) {
                        const uint2 x = Aq2[((size_t)(m0 + ml) * a.nblk + j) * 8 + ars * 4 + grp];
                        aop = (uint64_t)x.y << 32 | x.x;
                    }
                    const v4i d = mfma16(aop, bop);
                    const int me = mi * 4 + grp;
                    if (me < Mc) {
                        const size_t row = (size_t)(m0 + me);
                        int cs = HP ? d[0] * 256 + d[1] + d[2] * 128 : d[0];
                        if (BITS == 4) {
                            const int zp = (a.flags & kFlagZp) ? (int)a.Z[blk_index((int)n, j, a.nbg, 4)] : 8;
                            cs -= zp * a.Sq[row * a.nblk4 + j];
                        }
                        if (a.flags & kFlagDl) cs += (HP ? 256 : 1) * a.D[blk_index((int)n, j, a.nbg, JGh)];
                        if (DOTS) a.Cs[(row * a.N + n) * a.nblk + j] = cs;
                        else fbuf[me][j - j0][col] = (float)cs * sc;
                    }
                }
            }
        }
        if (!DOTS) {
            __syncthreads();
            if (cm < Mc) {
                const int jn = min(SEG, a.nblk - j0);
                const float* sa = a.Sa + (size_t)(m0 + cm) * a.nblk4 + j0;
                for (int jj = 0; jj < jn; ++jj) acc = __builtin_fmaf(sa[jj], fbuf[cm][jj][ccol], acc);
            }
            __syncthreads();
        }
    }
    if (!DOTS && cm < Mc) a.C[(size_t)(m0 + cm) * a.N + t * 16 + ccol] = acc;
}

// Activation records for the prefill GEMM: 4 lanes per (row, block) over
// Mpad rows and 2*nch blocks; padding rows and blocks quantize zeros.
template <bool HP>
__global__ __launch_bounds__(256) void quantize_rec_kernel(const float* __restrict__ A, int M, int K, int nblk,
                                                           int nch, int Mpad, uint8_t* __restrict__ R) {
    // A wave per (16-row tile, block j): lane (r, o) = (lane >> 2, lane & 3)
    // quantizes k-octet o of row r, the 4 lanes of a row one block, and
    // writes its 8 h bytes at pf_rec_byte(r, o) of the block's 1 KB and its
    // 8 l bytes 512 bytes later.  The wave fills the whole 1 KB.
    const int g = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int o = lane & 3, r = lane >> 2;
    const int nb2 = 2 * nch;
    const int mt = g / nb2, j = g - mt * nb2, m = 16 * mt + r;
    if (mt * 16 >= Mpad) return;  // whole waves only: the quad reductions need all lanes
    const bool valid = m < M && j < nblk;
    float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
    if (valid) {
        const float* src = A + (size_t)m * K + 32 * j + 8 * o;
        v0 = *reinterpret_cast<const float4*>(src);
        v1 = *reinterpret_cast<const float4*>(src + 4);
    }
    float s;
    uint2 ph, pl;
    quant4x8<HP>(v0, v1, s, ph, pl);
    uint8_t* rec = R + ((size_t)mt * nch + (j >> 1)) * kRecBytes;
    const int b = j & 1;
    *reinterpret_cast<uint2*>(rec + b * 1024 + pf_rec_byte(r, o)) = ph;
    *reinterpret_cast<uint2*>(rec + b * 1024 + 512 + pf_rec_byte(r, o)) = pl;
    if (o == 0) *reinterpret_cast<float*>(rec + kRecA + (b * 16 + r) * 4) = s;
}

// Row pairs per prefill workgroup: 32 rows for up to 32 rows, 64 for up to
// 64, otherwise 128.  `force` (BREEZE_HIP_PREFILL_RP) selects 1, 2 or 4 for
// tests.
int pick_pf_rp(int M, const char* force) {
    if (force) {
        const int v = std::atoi(force);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    return M <= 32 ? 1 : M <= 64 ? 2 : 4;
}

// Column tiles per workgroup for rp row pairs: among the instantiated
// widths, the one that minimizes (workgroup rounds at one workgroup per CU)
// x (tiles on the busiest SIMD, whose two waves hold column parts s / rp and
// (s + 4) / rp).  `force` (BREEZE_HIP_PREFILL_CT) selects an instantiated
// width for rp instead, for tests and tuning.
int pick_pf_ct(int ntiles, int gy, int rp, int n_cu, const char* force) {
    if (force) {
        const int v = std::atoi(force);
        for (const PfCfg& c : kPfCfgs)
            if (c.rp == rp && c.ct == v) return v;
    }
    int best = 0;
    long best_cost = -1;
    for (const PfCfg& c : kPfCfgs) {
        if (c.rp != rp) continue;
        const int parts = kPfWaves / rp, ctb = c.ct / parts, ctr = c.ct % parts;
        int simd = 0;
        for (int sm = 0; sm < 4; ++sm) {
            const int q0 = sm / rp, q1 = (sm + 4) / rp;
            simd = std::max(simd, 2 * ctb + (q0 < ctr) + (q1 < ctr));
        }
        const long wgs = (long)((ntiles + c.ct - 1) / c.ct) * gy;
        const long cost = (wgs + n_cu - 1) / n_cu * simd;
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = c.ct;
        }
    }
    return best;
}

// ------------------------------------------------------------------ RMSNorm
//
// The decoder's RMSNorm (kernel/qwen35_decoder.cpp:134-140), bit-identical:
// ss = sum of (double)x*x in element order, inv = 1/sqrtf((float)(ss/H) +
// eps), out = (x*inv)*w.  The sum is rebuilt exactly in parallel.  While the
// running sum s stays in one binade [2^e, 2^(e+1)), every partial sum is a
// multiple of u = 2^(e-52) and fl(s + t) = s + u*round(t/u), so such an
// element adds the integer k = round(t/u) whatever s is.  An element is
// "special" when that does not hold or is not certain: the first nonzero term
// (s = 0), a step that leaves the binade, an estimated partial sum within a
// relative 2^-20 of a power of two (exact specials), or an exact tie
// (t/u = n + 1/2, rounded to the even neighbour of s/u).  The estimates are a
// parallel prefix sum, within ~H*2^-53 (relative) of the true partial sums.
// A tie leaves s/u even, so a tie whose previous special is a tie adds
// X + (X & 1), X = (the k since that tie) + floor(t/u), whatever s is.  Only
// the "anchors" -- exact specials and the first tie after each -- need the
// running sum: one wave walks them in order, with everything between two
// anchors summed in parallel beforehand.  Rows with more than kNormMaxSpecial
// specials are summed in element order by wave 0 alone (one running sum,
// 64 terms squared at a time).  Rows up to kNormStage
// wide are staged in LDS and each thread holds its (at most kNormPer) terms
// and their classes in registers; wider rows are read from memory per pass.
constexpr int kNormThreads = 1024;
constexpr int kNormMaxSpecial = 1024;
constexpr int kNormStage = 8192;
constexpr int kNormPer = kNormStage / kNormThreads;
constexpr double kNormBand = 0x1p-20;

__device__ inline int ilogb_pos(double v) { return __builtin_amdgcn_frexp_exp(v) - 1; }

// v > 0 within a relative kNormBand of a power of two (either side).
__device__ inline bool near_pow2(double v) {
    const double m = __builtin_amdgcn_frexp_mant(v);  // [0.5, 1)
    return m < 0.5 * (1.0 + kNormBand) || m > 1.0 - kNormBand;
}


template <typename T>
__device__ inline T block_exclusive_scan(T v, T* wsum, T* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    T inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const T o = __shfl_up(inc, d);
        if (lane >= d) inc += o;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    T base = 0, all = 0;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) {
        if (i < wave) base += wsum[i];
        all += wsum[i];
    }
    *total = all;
    __syncthreads();
    return base + inc - v;
}

// 0 simple (k set), 1 exact special, 2 tie (k = floor(t/u)).
__device__ inline int norm_classify(double P, double t, unsigned long long* k) {
    *k = 0;
    if (t == 0.0) return 0;
    const double Q = P + t;
    if (P == 0.0 || near_pow2(P) || near_pow2(Q)) return 1;
    const int e = ilogb_pos(P);
    if (ilogb_pos(Q) != e) return 1;
    const double f = __builtin_ldexp(t, 52 - e);  // < 2^53: t < 2^(e+1)
    const double fl = __builtin_floor(f);
    *k = (unsigned long long)fl;
    const double fr = f - fl;
    if (fr == 0.5) return 2;
    if (fr > 0.5) *k += 1;
    return 0;
}

// Only (float)(ss / H) of the sum enters the output: the kernel first forms
// a tree sum of the squares (its thread's run, a 64-lane butterfly, the 16
// wave totals in order: at most per + 22 roundings per term) and lets
// norm_mean_from_bound decide; only when it cannot does it rebuild the
// in-order sum.
template <bool STAGED>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* __restrict__ X, const float* __restrict__ Wt,
                                                                int H, float eps, float* __restrict__ Out, int exact_only) {
    extern __shared__ float norm_row[];                      // STAGED: the row
    __shared__ double spec[kNormMaxSpecial];                 // t, or -(floor(t/u) + 1) for a tie
    __shared__ unsigned long long seg[kNormMaxSpecial + 1];  // sum of k with q specials before
    __shared__ unsigned long long gap[kNormMaxSpecial];      // non-anchor ties after anchor a
    __shared__ int alist[kNormMaxSpecial];                   // special index of anchor a
    __shared__ double wsum_d[kNormThreads / 64];
    __shared__ int wsum_i[kNormThreads / 64];
    __shared__ double ss_s;
    __shared__ float mean_s;  // (float)(ss / H)
    const float* xg = X + (size_t)blockIdx.x * H;
    float* o = Out + (size_t)blockIdx.x * H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int per = (H + kNormThreads - 1) / kNormThreads;

    // Shortcut: a tree sum T of the squares (elements tid + 1024 i, in
    // registers when STAGED; a 64-lane butterfly; the 16 wave totals in
    // order) and its error bound.  Any tree serves the bound, which needs
    // only its depth: at most per + 22 roundings per term.
    float xv[STAGED ? kNormPer : 1], wv[STAGED ? kNormPer : 1];
    double loc = 0.0;
    if constexpr (STAGED) {
#pragma unroll
        for (int i = 0; i < kNormPer; ++i) {
            const int j = tid + i * kNormThreads;
            xv[i] = j < H ? xg[j] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kNormPer; ++i) {
            const int j = tid + i * kNormThreads;
            wv[i] = j < H ? Wt[j] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kNormPer; ++i) loc += (double)xv[i] * (double)xv[i];
    } else {
        for (int j = tid; j < H; j += kNormThreads) loc += (double)xg[j] * (double)xg[j];
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) loc += __shfl_xor(loc, d);
    if (lane == 0) wsum_d[tid >> 6] = loc;
    __syncthreads();
    double T = 0.0;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) T += wsum_d[w];
    {
        float mean = 0.0f;
        // Uniform: every thread holds the same T.  NaN or inf totals (a
        // NaN or inf term; finite squares cannot overflow) take the long way.
        if (T - T == 0.0 && !exact_only && norm_mean_from_bound(T, H, per, &mean)) {
            const float inv = 1.0f / sqrtf(mean + eps);
            if constexpr (STAGED) {
#pragma unroll
                for (int i = 0; i < kNormPer; ++i) {
                    const int j = tid + i * kNormThreads;
                    if (j < H) o[j] = xv[i] * inv * wv[i];
                }
            } else {
#pragma unroll 4
                for (int j = tid; j < H; j += kNormThreads) o[j] = xg[j] * inv * Wt[j];
            }
            return;
        }
    }
    __syncthreads();  // wsum_d is reused below

    // The in-order reconstruction.
    if (STAGED) {
#pragma unroll
        for (int i = 0; i < kNormPer; ++i) {
            const int j = tid + i * kNormThreads;
            if (j < H) norm_row[j] = xv[i];
        }
        __syncthreads();
    }
    const float* x = STAGED ? norm_row : xg;
    const int j0 = min(tid * per, H), j1 = min(j0 + per, H);

    // STAGED: this thread's terms (0 past its range) and, after the
    // classification, their k and which of them are specials / ties.
    double tv[STAGED ? kNormPer : 1];
    unsigned long long kv[STAGED ? kNormPer : 1];
    unsigned smask = 0, tmask = 0;
    loc = 0.0;
    if constexpr (STAGED) {
#pragma unroll
        for (int i = 0; i < kNormPer; ++i) {
            const int j = j0 + i;
            const float xv = j < j1 ? x[j] : 0.0f;
            tv[i] = (double)xv * (double)xv;
            loc += tv[i];
        }
    } else {
        for (int j = j0; j < j1; ++j) loc += (double)x[j] * (double)x[j];
    }
    double tot_d;
    const double base = block_exclusive_scan<double>(loc, wsum_d, &tot_d);
    // Every thread holds the same total.  Squares of floats are at most
    // 2^256 and at most 2^31 of them cannot overflow a double, so the total
    // is NaN exactly when a term is (then the reference's sum is NaN too)
    // and +inf exactly when a term is and none is NaN (then its sum is +inf).
    const bool any_nan = tot_d != tot_d, any_inf = tot_d == __builtin_inf();
    if (any_nan || any_inf) {
        if (tid == 0) ss_s = any_nan ? __builtin_nan("") : __builtin_inf();
    } else {
        int cnt = 0;
        if constexpr (STAGED) {
            double P = base;
#pragma unroll
            for (int i = 0; i < kNormPer; ++i) {
                const int c = norm_classify(P, tv[i], &kv[i]);
                P += tv[i];
                smask |= (c != 0 ? 1u : 0u) << i;
                tmask |= (c == 2 ? 1u : 0u) << i;
            }
            cnt = __builtin_popcount(smask);
        } else {
            double P = base;
            for (int j = j0; j < j1; ++j) {
                const double t = (double)x[j] * (double)x[j];
                unsigned long long k;
                cnt += norm_classify(P, t, &k) != 0;
                P += t;
            }
        }
        int nspec;
        const int sbase = block_exclusive_scan<int>(cnt, wsum_i, &nspec);
        if (nspec <= kNormMaxSpecial) {
            for (int q = tid; q <= nspec; q += kNormThreads) seg[q] = 0;
            __syncthreads();
            if constexpr (STAGED) {
                int q = sbase;  // specials before element i
                unsigned long long run = 0;
#pragma unroll
                for (int i = 0; i < kNormPer; ++i) {
                    if (!((smask >> i) & 1u)) {
                        run += kv[i];
                        continue;
                    }
                    if (run) atomicAdd(&seg[q], run);
                    run = 0;
                    spec[q++] = (tmask >> i) & 1u ? -((double)kv[i] + 1.0) : tv[i];
                }
                if (run) atomicAdd(&seg[q], run);
            } else {
                double P = base;
                int q = sbase;  // specials before element j
                unsigned long long run = 0;
                for (int j = j0; j < j1; ++j) {
                    const double t = (double)x[j] * (double)x[j];
                    unsigned long long k;
                    const int c = norm_classify(P, t, &k);
                    P += t;
                    if (c == 0) {
                        run += k;
                        continue;
                    }
                    if (run) atomicAdd(&seg[q], run);
                    run = 0;
                    spec[q++] = c == 1 ? t : -((double)k + 1.0);
                }
                if (run) atomicAdd(&seg[q], run);
            }
            __syncthreads();
            // Anchors: special 0 (always exact: the first nonzero term),
            // every exact special, and every tie after an exact special.
            const int sper = (nspec + kNormThreads - 1) / kNormThreads;
            const int i0 = min(tid * sper, nspec), i1 = min(i0 + sper, nspec);
            int acnt = 0;
            for (int i = i0; i < i1; ++i) acnt += i == 0 || spec[i] >= 0.0 || spec[i - 1] >= 0.0;
            int nanch;
            const int abase = block_exclusive_scan<int>(acnt, wsum_i, &nanch);
            for (int q = tid; q < nanch; q += kNormThreads) gap[q] = 0;
            __syncthreads();
            {
                int a = abase - 1;  // anchor at or before special i
                unsigned long long run = 0;
                for (int i = i0; i < i1; ++i) {
                    if (i == 0 || spec[i] >= 0.0 || spec[i - 1] >= 0.0) {
                        if (run) atomicAdd(&gap[a], run);
                        run = 0;
                        alist[++a] = i;
                    } else {
                        const unsigned long long xq = seg[i] + (unsigned long long)(-spec[i]) - 1ull;
                        run += xq + (xq & 1ull);
                    }
                }
                if (run) atomicAdd(&gap[a], run);
            }
            __syncthreads();
            if (tid < 64) {
                // The walk, on all lanes of wave 0 alike: sd between binades,
                // S in units of 2^(e-52) within one.
                double sd = 0.0;
                long long S = 0;
                int e = 0;
                for (int a0 = 0; a0 < nanch; a0 += 64) {
                    long long sg = 0, gp = 0;
                    double v = 0.0;
                    if (a0 + tid < nanch) {
                        const int i = alist[a0 + tid];
                        sg = (long long)seg[i];
                        v = spec[i];
                        gp = (long long)gap[a0 + tid];
                    }
                    const int n = min(64, nanch - a0);
                    for (int l = 0; l < n; ++l) {
                        const double vl = __builtin_bit_cast(double, readlane64(__builtin_bit_cast(long long, v), l));
                        S += readlane64(sg, l);
                        if (vl < 0.0) {
                            S = (S + (long long)(-vl)) & ~1LL;  // -vl = floor(t/u) + 1
                        } else {
                            sd = __builtin_ldexp((double)S, e - 52) + vl;
                            e = ilogb_pos(sd);
                            S = (long long)__builtin_ldexp(sd, 52 - e);
                        }
                        S += readlane64(gp, l);
                    }
                }
                S += (long long)seg[nspec];
                if (tid == 0) ss_s = nspec ? __builtin_ldexp((double)S, e - 52) : 0.0;
            }
        } else if (tid < 64) {
            // Too many specials for the walk: wave 0 sums in element order.
            const double acc = norm_sumsq_inorder<64>(x, H);
            if (tid == 0) ss_s = acc;
        }
    }
    __syncthreads();
    if (tid == 0) mean_s = (float)(ss_s / (double)H);
    __syncthreads();
    const float inv = 1.0f / sqrtf(mean_s + eps);
    if constexpr (STAGED) {
#pragma unroll
        for (int i = 0; i < kNormPer; ++i) {
            const int j = tid + i * kNormThreads;
            if (j < H) o[j] = x[j] * inv * wv[i];
        }
    } else {
#pragma unroll 4
        for (int j = tid; j < H; j += kNormThreads) o[j] = x[j] * inv * Wt[j];
    }
}

// ------------------------------------------------------------------ argmax

__device__ inline unsigned long long block_max_key(unsigned long long k) {
    __shared__ unsigned long long red[256];
    red[threadIdx.x] = k;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + w]);
        __syncthreads();
    }
    return red[0];
}

constexpr int kArgmaxChunk = 4096;

// Partial keys over chunks of C (used after the rows kernel).
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ C, int N,
                                                             unsigned long long* __restrict__ part) {
    const int m = blockIdx.y, c = blockIdx.x;
    const int lo = c * kArgmaxChunk, hi = min(N, lo + kArgmaxChunk);
    unsigned long long best = 0;
    for (int i = lo + (int)threadIdx.x; i < hi; i += 256)
        best = max(best, argmax_key(C[(size_t)m * N + i], i));
    best = block_max_key(best);
    if (threadIdx.x == 0) part[(size_t)c * gridDim.y + m] = best;
}

// out = silu(g) * u elementwise (kernel/qwen35_decoder.cpp:128 and 408;
// silu_mul, the paired decode kernels' epilogue, so every path gives the
// reference's bits).  out may be u.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ g, const float* u, float* out,
                                                       size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = silu_mul(g[i], u[i]);
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const unsigned long long* __restrict__ part,
                                                           int nparts, int M, int64_t* __restrict__ out) {
    const int m = blockIdx.x;
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < nparts; i += 256) best = max(best, part[(size_t)i * M + m]);
    best = block_max_key(best);
    if (threadIdx.x == 0) out[m] = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
}

// ------------------------------------------------------------------ scratch
//
// Device scratch of the matmul calls: the stand-alone quantizers' activation
// records, the decode argmax state, argmax partials and the gate projection
// of the unpaired gate/up path.  Each (device, stream) pair owns its own
// scratch, so calls on different streams of one device never share it.  A
// buffer that has to grow is replaced and the old one is kept until the
// process ends, because a HIP graph captured earlier may still hold its
// address; growing is refused while the stream is capturing.

struct Scratch {
    hipStream_t stream = nullptr;
    uint8_t* aq = nullptr;  // [M][nblk][64] records of quantize_kernel
    float* sa = nullptr;    // [M][nblk4] block scales
    int* sq = nullptr;      // [M][nblk4] sums of q
    size_t aq_cap = 0, sa_cap = 0, sq_cap = 0;
    uint8_t* rec = nullptr;  // prefill activation records
    size_t rec_cap = 0;
    unsigned long long* parts = nullptr;  // argmax partial keys
    size_t parts_cap = 0;
    unsigned int* ticket = nullptr;  // decode argmax: ticket counter, then kDecMaxRows row keys; zero between calls
    float* gate = nullptr;           // gate projection of the unpaired gate/up path
    size_t gate_cap = 0;
    float* hn = nullptr;  // normalized rows when the norm runs as its own launch
    size_t hn_cap = 0;
    unsigned int* stick = nullptr;  // split-K: per-tile tickets, zero between calls
    size_t stick_cap = 0;
    float* sf = nullptr;  // split-K: per-tile block values and scales
    size_t sf_cap = 0;
    // Set for i4_matmul_noalloc_dev: the buffers above are carved from the
    // device's static scratch array and can never grow.
    bool fixed = false;
};

struct Workspace {
    std::mutex mu;  // held by every entry point while it uses this device's scratch
    std::vector<Scratch*> per_stream;
    std::vector<void*> retired;  // replaced scratch buffers (see above)
    float* hA = nullptr;  // device staging for the host-pointer entry points
    float* hC = nullptr;
    size_t hA_cap = 0, hC_cap = 0;
    hipStream_t stream = nullptr;
    int n_cu = 0;
    bool attr_set[1024] = {};  // decode kernel variants with the kernel attribute set
    bool dec8_attr[64] = {};  // the same for dec8_kernel, per (bits, mode) and (FUSE mode, metadata, LDS records)
    bool pf_attr[256] = {};
};

constexpr int kMaxDevices = 64;
Workspace g_ws[kMaxDevices];

// The scratch of `st` on this device; the caller holds w.mu.
Scratch* scratch_for(Workspace& w, hipStream_t st) {
    for (Scratch* s : w.per_stream)
        if (s->stream == st) return s;
    auto* s = new (std::nothrow) Scratch{};
    if (!s) {
        set_err("out of host memory");
        return nullptr;
    }
    s->stream = st;
    w.per_stream.push_back(s);
    return s;
}

// ------------------------------------------------------------------ no-allocation scratch
//
// i4_matmul_noalloc_dev takes all of its device scratch from `scratch`, a
// static array that every device holding this library keeps until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the symbol): each device's own address of
// it comes from hipGetSymbolAddress, once per device with that device
// current, and is kept in g_noalloc_ptr.  Layout per call: [0, 512) the
// decode argmax state (ticket and up to 32 row keys, cleared by a fill kernel on
// every call that uses it), then the activation records of this call (the
// stand-alone quantizer's records, scales and sums, or the prefill
// records), then the argmax partials.  Calls that overlap on one device
// share the array and race.
constexpr size_t kNoAllocBytes = 16u << 20;
constexpr size_t kNoAllocState = 512;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];
uint8_t* g_noalloc_ptr[kMaxDevices];

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int n, uint32_t v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
        (void)hipGetLastError();  // not left for the next launch check to find
        return true;
    }
    return cs != hipStreamCaptureStatusNone;
}

// Makes *p hold at least `need` elements for work on stream st.  A fixed
// scratch (the no-allocation entry point) never grows.
template <typename T>
bool grow(Workspace& w, hipStream_t st, T** p, size_t* cap, size_t need, const char* what, bool fixed = false) {
    if (need <= *cap) return true;
    if (fixed) {
        set_err("%s: this call needs %zu bytes of scratch in one buffer, more than the no-allocation entry "
                "point's fixed scratch holds for it (%zu bytes)",
                what, need * sizeof(T), *cap * sizeof(T));
        return false;
    }
    if (capturing(st)) {
        set_err("%s: this call needs %zu bytes of device scratch that the stream does not have yet, and "
                "memory cannot be allocated while the stream is capturing; make one call of this shape "
                "on the stream before capturing it",
                what, need * sizeof(T));
        return false;
    }
    const size_t n = std::max(need, *cap * 2);
    T* q = nullptr;
    if (!hip_ok(hipMalloc(reinterpret_cast<void**>(&q), n * sizeof(T)), what)) return false;
    if (*p) w.retired.push_back(*p);
    *p = q;
    *cap = n;
    return true;
}

bool ensure_quant(Workspace& w, Scratch& s, hipStream_t st, size_t rows, size_t nblk4) {
    const size_t n = rows * nblk4;
    return grow(w, st, &s.aq, &s.aq_cap, n * 64, "workspace alloc", s.fixed) &&
           grow(w, st, &s.sa, &s.sa_cap, n, "workspace alloc", s.fixed) &&
           grow(w, st, &s.sq, &s.sq_cap, n, "workspace alloc", s.fixed);
}

// ------------------------------------------------------------------ host helpers

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = 113;
            while (!(man & 0x400u)) {
                man <<= 1;
                --e;
            }
            bits = sign | (uint32_t)e << 23 | (man & 0x3FFu) << 13;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | man << 13 | (man ? 0x00400000u : 0u);
    } else {
        bits = sign | (exp + 112u) << 23 | man << 13;
    }
    float f;
    std::memcpy(&f, &bits, sizeof f);
    return f;
}

// Builds a handle from a canonical host representation:
//   raw: MatMulNBits bytes [N][nblk][16 or 32] (INT8 unsigned w+128, or
//        already signed with raw_signed); scales fp32 [N][nblk];
//   zp:  INT4 zero points [N][nblk] or empty; delta: legacy [N][nblk] or empty.
void* build_handle(const uint8_t* raw, bool raw_signed, const float* scales, int N, int K,
                   int bits, const std::vector<int8_t>& zp, const std::vector<int32_t>& delta) {
    const int nblk = K / 32;
    const int JG = bits == 8 ? 2 : 4;
    const int nbg = (nblk + JG - 1) / JG;
    const int nblk_pad = nbg * JG;
    const int nblk4 = (nblk + 3) / 4 * 4;

    // Repeated scales are stored once: per column, or per aligned group of
    // 2^k blocks (bitwise comparison, so every value is kept as given).
    int sc_shift = 31, ngrp = 1, sc_group = 0;
    {
        bool per_col = true;
        for (int n = 0; n < N && per_col; ++n)
            for (int j = 1; j < nblk; ++j)
                if (std::memcmp(&scales[(size_t)n * nblk + j], &scales[(size_t)n * nblk], 4)) {
                    per_col = false;
                    break;
                }
        if (!per_col) {
            for (int sh = 6; sh >= 0; --sh) {
                const int G = 1 << sh;
                bool ok = true;
                for (int n = 0; n < N && ok; ++n)
                    for (int j = 0; j < nblk; ++j)
                        if (std::memcmp(&scales[(size_t)n * nblk + j],
                                        &scales[(size_t)n * nblk + (j & ~(G - 1))], 4)) {
                            ok = false;
                            break;
                        }
                if (ok) {
                    sc_shift = sh;
                    ngrp = (nblk + G - 1) / G;
                    sc_group = G;
                    break;
                }
            }
        }
    }
    // Handles with explicit zero points, a legacy corr, or scale groups
    // smaller than a chunk keep all three per-block arrays, so the decode
    // kernel's loads stay unconditional.
    const bool extra = !zp.empty() || !delta.empty() || (sc_shift != 31 && (1 << sc_shift) < JG);
    std::vector<float> sc_dev;
    if (extra) {
        sc_dev.assign((size_t)N * nblk_pad, 0.0f);
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < nblk; ++j) sc_dev[blk_index(n, j, nbg, JG)] = scales[(size_t)n * nblk + j];
    } else {
        sc_dev.resize((size_t)N * ngrp);
        for (int n = 0; n < N; ++n)
            for (int gi = 0; gi < ngrp; ++gi)
                sc_dev[grp_index(n, sc_shift == 31 ? 0 : gi << sc_shift, ngrp, sc_shift)] =
                    scales[(size_t)n * nblk + (sc_shift == 31 ? 0 : (gi << sc_shift))];
    }
    std::vector<int8_t> zp_dev;
    if (extra && bits == 4) {
        zp_dev.assign((size_t)N * nblk4, 8);
        if (!zp.empty())
            for (int n = 0; n < N; ++n)
                for (int j = 0; j < nblk; ++j) zp_dev[blk_index(n, j, nbg, 4)] = zp[(size_t)n * nblk + j];
    }
    std::vector<int32_t> dl_dev;
    if (extra) {
        dl_dev.assign((size_t)N * nblk_pad, 0);
        if (!delta.empty())
            for (int n = 0; n < N; ++n)
                for (int j = 0; j < nblk; ++j) dl_dev[blk_index(n, j, nbg, JG)] = delta[(size_t)n * nblk + j];
    }

    auto* h = new (std::nothrow) Handle{};
    if (!h) {
        set_err("out of host memory");
        return nullptr;
    }
    h->magic = kMagic;
    h->N = N;
    h->K = K;
    h->nblk = nblk;
    h->bits = bits;
    h->nbg = nbg;
    h->nblk_pad = nblk_pad;
    h->nblk4 = nblk4;
    h->sc_shift = sc_shift;
    h->ngrp = ngrp;
    h->sc_group = sc_group;
    h->sc_blk = extra;
    h->has_zp = !zp.empty();
    h->has_dl = !delta.empty();
    h->extra = extra;
    (void)hipGetDevice(&h->device);

    const size_t wbytes = (size_t)(N / 16) * nbg * 64 * 16;
    const size_t rawbytes = (size_t)N * nblk * 4 * bits;
    uint8_t* draw = nullptr;
    bool ok = hip_ok(hipMalloc(&h->W, wbytes), "weight alloc") &&
              hip_ok(hipMalloc(&h->S, sc_dev.size() * 4), "scale alloc") &&
              (zp_dev.empty() || hip_ok(hipMalloc(&h->Z, zp_dev.size()), "zero-point alloc")) &&
              (dl_dev.empty() || hip_ok(hipMalloc(&h->D, dl_dev.size() * 4), "corr alloc")) &&
              hip_ok(hipMalloc(&draw, rawbytes), "staging alloc");
    ok = ok && hip_ok(hipMemcpy(draw, raw, rawbytes, hipMemcpyHostToDevice), "weight upload") &&
         hip_ok(hipMemcpy(h->S, sc_dev.data(), sc_dev.size() * 4, hipMemcpyHostToDevice), "scale upload") &&
         (zp_dev.empty() ||
          hip_ok(hipMemcpy(h->Z, zp_dev.data(), zp_dev.size(), hipMemcpyHostToDevice), "zero-point upload")) &&
         (dl_dev.empty() ||
          hip_ok(hipMemcpy(h->D, dl_dev.data(), dl_dev.size() * 4, hipMemcpyHostToDevice), "corr upload"));
    if (ok) {
        const size_t total = (size_t)(N / 16) * nbg * 64;
        const unsigned blocks = (unsigned)((total + 255) / 256);
        repack_kernel<<<blocks, 256>>>(draw, h->W, N, nblk, nbg, bits, raw_signed ? 1 : 0);
        ok = hip_ok(hipGetLastError(), "repack launch");
        if (ok && bits == 8) {
            const size_t n_ws = (size_t)(N / 16) * nbg * 16;
            ok = hip_ok(hipMalloc(&h->WS, n_ws * 2 * sizeof(int32_t)), "weight-sum alloc");
            if (ok) {
                wsum_kernel<<<(unsigned)((n_ws + 255) / 256), 256>>>(h->W, h->WS, N / 16, nbg);
                ok = hip_ok(hipGetLastError(), "weight-sum launch");
            }
        }
        ok = ok && hip_ok(hipDeviceSynchronize(), "repack");
    }
    if (draw) (void)hipFree(draw);
    if (!ok) {
        if (h->W) (void)hipFree(h->W);
        if (h->S) (void)hipFree(h->S);
        if (h->Z) (void)hipFree(h->Z);
        if (h->D) (void)hipFree(h->D);
        if (h->WS) (void)hipFree(h->WS);
        delete h;
        return nullptr;
    }
    h->dev_bytes = wbytes + sc_dev.size() * 4 + zp_dev.size() + dl_dev.size() * 4 +
                   (h->WS ? (size_t)(N / 16) * nbg * 16 * 2 * 4 : 0);
    return h;
}

void fill_args(const Handle* h, GemvArgs& a, int M) {
    a.W = h->W;
    a.S = h->S;
    a.Z = h->Z;
    a.D = h->D;
    a.M = M;
    a.N = h->N;
    a.K = h->K;
    a.nblk = h->nblk;
    a.nblk4 = h->nblk4;
    a.nbg = h->nbg;
    a.nblk_pad = h->nblk_pad;
    a.sc_shift = h->sc_shift;
    a.ngrp = h->ngrp;
    a.flags = h->extra ? ((h->Z ? kFlagZp : 0) | kFlagDl | kFlagScBlk) : 0;
    a.ntiles = h->N / 16;
}

// ------------------------------------------------------------------ routing
//
// plan_call decides, from the handle's shape and the call alone, which kernel
// serves a call and how it is launched; run() launches what the plan says
// (i4_plan_query exposes the plan to tests).  Every threshold below is a
// measured crossover on MI355X, in one table, with the measurement behind it
// (us per call, before -> after the choice made):
//
//   kFusedMaxBlocks2 (768 row-blocks: rows x 32-blocks of K; one or two
//   rows) and kFusedMaxBlocks (512; more rows)  the decode prologue
//   quantizes the activation itself up to here (passes of 256 row-blocks
//   over the sixteen waves); past it the stand-alone quantizer stages
//   records.  Staged -> fused: W4 K=12288 N=4096 at 2 rows (768) 9.75 ->
//     9.07, W4 K=17408 at 1 row (544) N=64 9.14 -> 8.43, N=5120 15.79 ->
//     14.80; W4 K=5120 N=17408 at 4 rows (640) 15.09 -> 15.13; past them,
//     W4 K=17408 N=64 at 2 rows (1088) 10.38 -> 10.76, W4 K=12288 N=4096 at
//     3 / 4 / 8 rows (1152 / 1536 / 2 x 1536) 10.39 / 10.40 / 12.96 ->
//     11.11 / 12.27 / 16.56: each pass of 256 row-blocks costs ~0.55 us on
//     every CU.
//   kNormFusedMaxBlocks (384)  the same with the RMSNorm in the prologue:
//     q/k/v at K = 5120, 3 rows (480 row-blocks): 16.6 fused against 15.4
//     for the norm kernel then the projections; 2 rows even.
//   dec_max_rows  most rows the decode kernels take before the prefill GEMM
//     does, falling with the width (the GEMM spreads more column tiles over
//     the CUs, every decode row group re-reads the weights; INT8 moves twice
//     the bytes per weight).  GEMM -> decode at 12 / 16 rows: W4 K=12288
//     N=4096 119 -> 21 / 120 -> 22, W8 K=5120 N=5120 40 -> 17 / 40 -> 18; at
//     20 / 32 rows: W4 K=12288 N=4096 119 -> 28 / 120 -> 37, W8 K=12288
//     N=4096 87 -> 43 / 88 -> 50, W4 K=4096 N=12288 44 -> 29 / 44 -> 42, W4
//     K=5120 N=17408 56 -> 42 / 56 -> 63, W8 K=4096 N=12288 34 -> 40 / 35 ->
//     51; W8 K=5120 N=17408 at 16 rows 42 -> 46.  With the eight-row groups
//     (which read the weights half as often) the limit rises on two widths:
//     W8 K=5120 N=17408 (1088 tiles) at 16 rows 41.4 -> 35.4 (24 rows: 42.7
//     -> 46.9), W4 K=5120 N=17408 at 32 rows 53.5 -> 46.7; it stays on W8
//     K=5120 N=151936 (16 rows: 180 -> 244), W8 K=4096 N=12288 (24 rows:
//     32.9 -> 45.8), W4 K=5120 N=27648 (32 rows: 54.5 -> 69.2).  From 2048
//     W8 tiles the GEMM takes 9 rows and more: K=5120 N=151936 at 9 / 12
//     rows 193.8 / 188.8 against 245.2 / 247.1, K=4096 N=151936 159.0 /
//     159.7 against 253.9 / 253.4, K=5120 N=65536 99.7 / 100.6 against
//     111.1 / 111.3.  W4 past 1536 tiles stops at 16 rows on the eight-row
//     groups: K=5120 N=151936 at 16 / 24 rows 191.6 / 293.0 against the
//     GEMM's 277.0 / 285.3, N=65536 90.7 / 128.3 against 97.5 / 101.5.
//   kPairMaxRows4 (16)  paired and multi-projection calls on the four-row
//     groups (kDec8MaxRows, 32, on the eight-row groups).
//   dec8_prologue_call  where the four-row groups quantize in their own
//     prologue (K <= 4096 at 4 rows), the eight-row groups' stand-alone
//     quantizer costs a launch; they take such calls from 24 rows, from 12
//     rows with K >= 3072, and from 8 rows with K >= 4096 over 768 tiles or
//     more (four-row -> eight-row): W8 K=3072 N=8192 at 12 / 24 rows 15.3 /
//     25.1 -> 12.3 / 16.9, W4 K=4096 N=12288 at 16 / 32 rows 20.6 / 36.2 ->
//     17.4 / 27.6, W4 K=2048 N=8192 at 12 / 24 rows 9.05 / 14.3 -> 11.3 /
//     13.0; at 8 rows W8 K=N=4096 9.4 -> 12.1 (kept on the four-row groups),
//     W8 K=4096 N=12288 18.5 -> 14.7, W4 13.2 -> 13.1.  Elsewhere (staged
//     records) the eight-row groups take 5-32 rows: W4 K=12288 N=4096 at 8 /
//     16 / 32 rows 13.6 / 21.1 / 34.0 -> 13.1 / 18.6 / 29.2, W8 K=12288
//     N=4096 at 24 rows 49.3 -> 34.3, W4 K=17408 N=5120 at 16 rows 54.0 ->
//     30.6, at 9 / 12 rows W4 K=17408 N=5120 40.1 / 44.9 -> 26.9 / 27.1, W8
//     K=5120 N=5120 16.4 / 16.4 -> 12.5 / 12.7 (W4 K=5120 N=5120 13.3 / 13.5
//     -> 13.9 / 13.3, the one loss seen).
//   kDec8LrecTiles (2)  the eight-row groups copy their records into LDS
//     when the busiest workgroups have this many tiles: W8 K=5120 N=151936
//     at 5 / 8 rows 173.7 / 171.9 -> 152.9 / 154.1, W8 K=5120 N=17408 at 8 /
//     16 rows 25.0 / 34.6 -> 23.3 / 31.2.
//   kPrefillMinRows (9)  the prefill GEMM takes what the decode kernels do
//     not, from 9 rows (not with a legacy corr; the rows kernel serves those
//     and the block-integer export).
//   pick_pf_rp  32-row prefill workgroups up to 32 rows, 64 up to 64, then
//     128 (the C4 shape's 512 rows fill the CUs with 128-row workgroups).
//   kStreamIdleDiv (8)  plain decode calls read their weight chunks with
//     non-temporal loads when at most one in 8 of a tile's producer slots
//     (15 a phase) is idle.  Weights are read once a call; the hint streams
//     them faster (a plain copy kernel over 1 GiB: 6.0-6.4 -> 7.0-7.2 TB/s),
//     but the idle slots' loads, which re-read a tile's last chunk or warm
//     L2 for the next tile's, then miss more.  Plain -> non-temporal: idle
//     1/10-1/9 of the slots (W4 K=12288, W8 and W4 K=5120): C3 M=1 7.89 ->
//     7.47, W8 K=5120 N=151936 (C5) 134.1 -> 122.8, N=17408 19.05 -> 17.57,
//     N=16384 16.68 -> 15.61, W4 K=5120 N=17408 11.70 -> 11.53, W4 K=17408
//     N=5120 14.97 -> 14.74; idle 11/75 (W8 K=4096): N=4096 (C1) 4.89 ->
//     5.39, N=8192 7.74 -> 7.42, N=12288 10.56 -> 9.99; idle 13/45 (W4
//     K=4096): N=12288 (C2) 7.19 -> 7.31, N=24576 12.39 -> 13.16, N=32768
//     16.0 -> 15.9, N=65536 35.5 -> 35.2.  Eight-row groups (14 chunks a
//     phase), kStreamMaxGroups (2): W4 K=12288 N=4096 at 8 / 16 / 24 rows
//     (one / two / three row groups) 13.13 / 19.12 / 29.75 -> 12.65 / 18.99 /
//     31.79, W8 K=5120 N=17408 at 16 rows 33.13 -> 31.27, W4 28.77 -> 28.50.
//   flow_phases  plain decode calls whose workgroups hold two tiles or more
//     of at least 15 whole chunks that do not fill whole phases run their
//     phases across tile boundaries (one stream of chunks), which leaves
//     few idle slots, so the non-temporal rule above counts over the
//     stream.  Plain -> flow with non-temporal loads: W4 K=4096 N=12288
//     (C2) 7.22 -> 6.98, N=24576 12.25 -> 11.3, W8 K=4096 N=12288 10.5 ->
//     9.8, W8 K=5120 N=17408 18.9 -> 17.2, N=151936 (C5, with non-temporal
//     loads before) 122.7 -> 119.3; W4 K=5120 N=17408 and K=17408 N=5120
//     even.  One tile a workgroup (W4 K=17408 N=64, forced): 8.30 -> 8.63.
//     The gate/up pair's stream alternates each column tile's gate and up
//     chunks (two stream tiles a column tile): W4 K=5120 N=17408 at 1 / 2 /
//     4 rows 23.0 / 22.8 / 25.6 -> 21.8 / 21.8 / 24.3 (with non-temporal
//     loads, which the pair takes only with its phases across tiles).
//   kSplitMaxTiles (8), kSplitMinPhases (20)  split-K takes plain decode
//     calls of at most 8 column tiles whose tiles have 20 phases or more
//     (15 chunks a phase: W8 K >= 18272, W4 K >= 36512).  The unsplit
//     kernel spends ~0.45 (W8) / ~0.68 (W4) us a phase on one CU; the split
//     launch spends ~3 us handing the pieces' block values across CUs
//     (device-scope stores, a ticket, device-scope loads) and folds nblk
//     blocks on one wave.  64 columns, one row, unsplit -> split: W8 K=12288
//     / 17408 / 24576 / 32768 7.65 / 10.12 / 12.96 / 17.10 -> 8.91 / 10.17 /
//     11.98 / 13.92; W4 K=24576 / 32768 10.26 / 14.20 -> 12.76 / 13.97; two
//     rows: W8 K=17408 11.94 -> 11.48, W4 K=17408 10.51 -> 12.71; W4
//     K=32768 N=256 (16 tiles, 256 pieces) 14.46 -> 16.33; W4 K=4096 N=1024
//     3.81 -> 8.41.
//
// Environment overrides for tests and tuning: BREEZE_HIP_DEC_ROWS (decode
// row limit), BREEZE_HIP_DEC8 (0: never the eight-row groups; 2: they take
// every prologue-quantized call), BREEZE_HIP_DEC8_ROWS (their row limit),
// BREEZE_HIP_DEC8_LREC (0: records never in LDS; n: from n tiles),
// BREEZE_HIP_PREFILL_RP / _CT (prefill workgroup shape), BREEZE_HIP_FUSED_MAX_BLOCKS
// (row-blocks the decode prologue quantizes), BREEZE_HIP_SPLIT (split-K),
// BREEZE_HIP_STREAM (non-temporal weight loads), BREEZE_HIP_FLOW (phases
// across tile boundaries).
constexpr int kFusedMaxBlocks = 512, kFusedMaxBlocks2 = 768;
constexpr int kFusedCapBlocks = kQuantPasses * 256;  // what the prologue can quantize
constexpr int kDecMaxRows = 32, kDecMaxGroups = 8;
constexpr int kDec8MaxRows = 32;  // four row groups of eight
constexpr int kPairMaxRows4 = 16;
constexpr int kDec8LrecTiles = 2;
constexpr int kPrefillMinRows = 9;
constexpr int kSplitMaxTiles = 8, kSplitMinPhases = 20;
constexpr int kStreamIdleDiv = 8, kStreamMaxGroups = 2;

// Row-blocks the decode prologue quantizes itself for calls of M rows
// (BREEZE_HIP_FUSED_MAX_BLOCKS sets it for every M, up to kFusedCapBlocks).
int fused_max_blocks(int M) {
    if (const char* v = std::getenv("BREEZE_HIP_FUSED_MAX_BLOCKS")) {
        const int b = std::atoi(v);
        if (b >= 0) return std::min(b, kFusedCapBlocks);
    }
    return M <= 2 ? kFusedMaxBlocks2 : kFusedMaxBlocks;
}

int dec_max_rows(int bits, int ntiles, bool eight, const char* force) {
    if (force) {
        const int v = std::atoi(force);
        if (v >= 1 && v <= kDecMaxRows) return v;
    }
    if (bits == 8) return ntiles >= 2048 ? 8 : ntiles >= 1024 ? (eight ? 16 : 12) : ntiles > 512 ? 16 : 32;
    if (eight) return ntiles > 1536 ? 16 : 32;
    return ntiles > 768 ? 24 : 32;
}

// Whether the eight-row groups take a call the four-row groups would quantize
// in their own prologue (see dec8_prologue_call above).
bool dec8_prologue_call(int M, int nblk, int ntiles) {
    const char* d8 = std::getenv("BREEZE_HIP_DEC8");
    return M >= 24 || (M >= 12 && nblk >= 96) || (M >= 8 && nblk >= 128 && ntiles >= 768) || (d8 && d8[0] == '2');
}

// What routing reads of a handle.
struct Shape {
    int bits, N, nblk, nblk4, nblk_pad;
    bool extra, has_dl, has_ws;
};
Shape shape_of(const Handle* h) {
    return Shape{h->bits, h->N, h->nblk, h->nblk4, h->nblk_pad, h->extra, h->has_dl, h->WS != nullptr};
}

// LDS bytes of the decode kernel for Mr_max rows per row group, or 0 if the
// activation records of a row group do not fit (in LDS, or in the
// prologue's 6-uint4-per-thread record copy).
int plan_dec_lds(int nblk, int Mr_max, int JG, bool p64 = false) {
    if (Mr_max * nblk > kFusedCapBlocks && Mr_max * nblk * 4 > 6 * kDecWaves * 64) return 0;
    const int total = dec_lds(Mr_max, nblk, JG, p64).total;
    return total <= kLdsMax ? total : 0;
}

template <int BITS, bool HP>
hipError_t launch_rows_bits(const GemvArgs& a, dim3 grid, bool dots, hipStream_t st) {
    if (dots) rows_kernel<BITS, HP, true><<<grid, kRowWaves * 64, 0, st>>>(a);
    else rows_kernel<BITS, HP, false><<<grid, kRowWaves * 64, 0, st>>>(a);
    return hipGetLastError();
}

int device_cus(Workspace& w, int dev) {
    if (w.n_cu == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        w.n_cu = n;
    }
    return w.n_cu;
}

int dec8_lrec_min_tiles() {
    if (const char* v = std::getenv("BREEZE_HIP_DEC8_LREC")) {
        const int t = std::atoi(v);
        return t > 0 ? t : std::numeric_limits<int>::max();
    }
    return kDec8LrecTiles;
}
// Rows of the eight-row groups that take M rows (M rounded up to 8).
int dec8_rows(int M) { return (M + kRows8 - 1) / kRows8 * kRows8; }
// Whether the decode kernel in row groups of eight can take a call: one
// without the block-integer export, with its eight rows' block scales and
// sums within two uint4 per thread and its LDS plan within the limit.
bool dec8_takes(const Shape& h, int M, bool dots) {
    int max_rows = kDec8MaxRows;
    if (const char* r = std::getenv("BREEZE_HIP_DEC8_ROWS")) max_rows = std::min(kDec8MaxRows, std::max(5, std::atoi(r)));
    if (M < 5 || M > max_rows || dots) return false;
    const char* f = std::getenv("BREEZE_HIP_DEC8");
    if (f && f[0] == '0') return false;
    if ((size_t)kRows8 * h.nblk4 / 4 > 2 * (size_t)kDecWaves * 64) return false;
    return dec8_lds(h.nblk, h.bits == 8 ? 2 : 4).total <= kLdsMax;
}

// The kernel that serves a call.
enum Route { kRouteNone = 0, kRouteDec = 1, kRouteDec8 = 2, kRoutePrefill = 3, kRouteRows = 4 };
// The stand-alone quantizer launched ahead of it: none (the decode prologue
// quantizes), records for the four-row groups or the rows kernel, records in
// the eight-row groups' operand order, or the prefill GEMM's records.
enum Quant { kQuantNone = 0, kQuantStaged = 1, kQuantRows8 = 2, kQuantPrefill = 3 };

struct CallKind {
    bool dots = false;    // block-integer export
    bool argmax = false;  // per-row argmax
    bool pair = false;    // gate/up pair in one launch
    bool multi = false;   // several projections in one launch
    bool norm = false;    // multi with the RMSNorm in the prologue
    int tiles = 0;        // column tiles of the launch (all segments of a multi call)
};

struct Plan {
    int route = kRouteNone;  // kRouteNone: a paired or multi call no decode launch takes
    int quant = kQuantNone;
    bool fused = false;      // the decode prologue quantizes
    bool p64 = false;        // decode, one or two rows: block pairs on 16x16x64
    bool lrec = false;       // eight-row groups: records in LDS
    int rs = 4;              // rows per row group
    int RG = 1, NG = 1;      // row groups, tile ranges
    int pair_xcd = 0;        // the row groups of a tile range share an XCD
    int lds = 0;             // dynamic LDS bytes (decode kernels)
    int pf_rp = 0, pf_ct = 0, Mpad = 0;  // prefill: row pairs, column tiles, padded rows
    int grid_x = 0, grid_y = 1;
    int split = 0;           // decode split-K: workgroups per tile (0: none)
    bool stream = false;     // decode: weight chunks read with non-temporal loads
    bool flow = false;       // decode: phases run across the tiles of a workgroup
};

// Phases across tile boundaries (kFuseFlow) for a plain decode call whose
// busiest workgroups hold two tiles or more of at least 15 whole chunks
// (no padded last chunk) that do not fill whole phases (see the routing
// table).  BREEZE_HIP_FLOW=0 / 1
// turns it off / on wherever it applies.
bool flow_phases(const Shape& h, const CallKind& k, const Plan& p, int tiles) {
    if (k.multi || k.norm || k.dots || p.split) return false;
    const int JG = h.bits == 8 ? 2 : 4;
    const int nbg = (h.nblk + JG - 1) / JG;
    if (nbg < kProducers || h.nblk % JG) return false;  // one tile end a phase; no padded chunk
    const int per_wg = (tiles + p.NG - 1) / p.NG * (k.pair ? 2 : 1);  // tiles of the stream
    if (const char* env = std::getenv("BREEZE_HIP_FLOW")) return env[0] == '1';
    return per_wg >= 2 && nbg % kProducers != 0;
}

// Non-temporal weight loads (kFuseStream) for a plain decode call whose
// tiles leave at most one in kStreamIdleDiv producer slots idle
// (`producers` chunks a phase: the last phase's empty slots re-read or
// prefetch chunks through L2, which non-temporal fills serve worse) and
// whose tiles are read by at most kStreamMaxGroups row groups (more share
// the weights through L2); see the routing table.  BREEZE_HIP_STREAM=0 / 1
// turns them off / on for every plain decode call.
bool stream_loads(const Shape& h, const CallKind& k, const Plan& p, int producers, int tiles) {
    // A gate/up pair reads non-temporally only with its phases across tiles.
    if ((k.pair && !p.flow) || k.multi || k.norm || k.dots || p.split) return false;
    if (const char* env = std::getenv("BREEZE_HIP_STREAM")) return env[0] == '1';
    const int JG = h.bits == 8 ? 2 : 4;
    int nbg = (h.nblk + JG - 1) / JG;
    if (p.flow) nbg *= (tiles + p.NG - 1) / p.NG * (k.pair ? 2 : 1);  // one stream over the busiest workgroup's tiles
    const int slots = (nbg + producers - 1) / producers * producers;
    return p.RG <= kStreamMaxGroups && (slots - nbg) * kStreamIdleDiv <= slots;
}

// Split-K for a plain decode call of at most four rows (one row group): the
// workgroups per tile (S pieces of the tile's phases), or 0.  S fills the
// CUs, at most one phase a piece.  A piece's LDS holds only its own blocks,
// so any K fits whose rows of a piece fit one prologue and whose fold
// staging fits the LDS; *lds receives the launch's LDS bytes.  Taken by
// default for tall-skinny calls: at most kSplitMaxTiles tiles and at least
// kSplitMinPhases phases a tile (see the routing table).  BREEZE_HIP_SPLIT:
// 0 never, 1 wherever it fits, n >= 2 forces n pieces (at most one per
// phase).
int split_pieces(const Shape& h, int M, const CallKind& k, int n_cu, int* lds) {
    if (M > 4 || k.dots || k.argmax || k.pair || k.multi || k.norm) return 0;
    const int JG = h.bits == 8 ? 2 : 4;
    const int ntiles = h.N / 16;
    const int nbg = (h.nblk + JG - 1) / JG;
    const int npw = (nbg + kProducers - 1) / kProducers;
    if (npw < 2) return 0;
    int S = std::min(npw, n_cu / ntiles);
    const char* env = std::getenv("BREEZE_HIP_SPLIT");
    const int force = env ? std::atoi(env) : -1;
    if (force == 0) return 0;
    if (force >= 2) S = std::min(force, npw);
    else if (force != 1 && (ntiles > kSplitMaxTiles || npw < kSplitMinPhases)) return 0;
    if (S < 2) return 0;
    const int lblk = split_piece_blocks(npw, S, nbg, JG);
    if (M * std::min(lblk, h.nblk) > kFusedCapBlocks) return 0;
    const int total = dec_lds(M, lblk, JG, M <= 2).total;
    const int need = split_flag_off(M, h.nblk4, total) + 16;
    if (need > kLdsMax) return 0;
    *lds = need;
    return S;
}

Plan plan_call(const Shape& h, int M, const CallKind& k, int n_cu) {
    Plan p;
    const int JG = h.bits == 8 ? 2 : 4;
    const int ntiles = h.N / 16;
    int split_lds = 0;
    if (const int S = split_pieces(h, M, k, n_cu, &split_lds)) {
        // Split-K: one row group, the prologue quantizes each piece.
        p.route = kRouteDec;
        p.fused = true;
        p.p64 = M <= 2;
        p.rs = 4;
        p.NG = ntiles;
        p.grid_x = ntiles * S;
        p.lds = split_lds;
        p.split = S;
        return p;
    }
    const bool fz = k.pair || k.multi;
    int Mr_max = std::min(M, 4);
    // One or two rows: block pairs per MFMA when that record layout fits.
    const int lds_p64 = (M <= 2 && !k.dots) ? plan_dec_lds(h.nblk, Mr_max, JG, true) : 0;
    p.p64 = lds_p64 > 0;
    // Past four rows the row groups quantize in their prologue only when
    // four rows of K fit one prologue's blocks; otherwise the eight-row
    // groups take the call if they can.
    const int fused_max = fused_max_blocks(M);
    const bool eight = 4 * h.nblk > fused_max_blocks(4) && dec8_takes(h, kRows8, k.dots);
    const int dec_rows = std::min(fz ? (eight ? kDec8MaxRows : kPairMaxRows4) : kDecMaxRows,
                                  dec_max_rows(h.bits, ntiles, eight, std::getenv("BREEZE_HIP_DEC_ROWS")));
    int lds = p.p64 ? lds_p64 : (M <= dec_rows && !k.dots) ? plan_dec_lds(h.nblk, Mr_max, JG) : 0;
    // Rows per row group: 4, or 2 or 1 where four rows of records do not
    // fit (long K: the staged copy holds 1536 row-blocks, so two rows reach
    // K = 24576 and one row K = 49152).  Eight row groups at most.
    int rs = 4;
    for (int r = 2; r >= 1 && !lds; r >>= 1) {
        if (r >= Mr_max) continue;  // that plan did not fit
        if (M > std::min(dec_rows, r * kDecMaxGroups) || k.dots || fz) break;
        lds = plan_dec_lds(h.nblk, r, JG);
        if (lds) {
            rs = r;
            Mr_max = r;
        }
    }
    const bool dec = lds > 0;
    if (k.multi && (h.extra || k.argmax)) return p;
    const bool fused = dec && Mr_max * h.nblk <= fused_max;
    const bool dec8 = M <= dec_rows && (!fused || dec8_prologue_call(M, h.nblk, ntiles)) && !k.norm &&
                      dec8_takes(h, M, k.dots);
    if (fz && !(dec8 || (dec && M <= kPairMaxRows4))) return p;
    if (k.norm && !(fused && Mr_max * h.nblk <= kNormFusedMaxBlocks)) return p;
    const bool pre = !dec && !dec8 && !k.dots && M >= kPrefillMinRows && (h.bits == 4 || h.has_ws) && !h.has_dl;
    const int tiles = k.tiles > 0 ? k.tiles : ntiles;
    p.fused = fused;
    if (pre) {
        p.route = kRoutePrefill;
        p.quant = kQuantPrefill;
        p.pf_rp = pick_pf_rp(M, std::getenv("BREEZE_HIP_PREFILL_RP"));
        const int rows = 32 * p.pf_rp;
        p.Mpad = (M + rows - 1) / rows * rows;
        p.grid_y = p.Mpad / rows;
        p.pf_ct = pick_pf_ct(tiles, p.grid_y, p.pf_rp, n_cu, std::getenv("BREEZE_HIP_PREFILL_CT"));
        p.grid_x = (tiles + p.pf_ct - 1) / p.pf_ct;
    } else if (dec8) {
        p.route = kRouteDec8;
        p.quant = kQuantRows8;
        p.rs = kRows8;
        p.RG = dec8_rows(M) / kRows8;
        p.NG = std::min(tiles, std::max(1, n_cu / p.RG));
        p.pair_xcd = (p.RG > 1 && p.NG % 8 == 0) ? 1 : 0;
        p.grid_x = p.NG * p.RG;
        // Records in LDS where the busiest workgroups have several tiles (or
        // paired tiles) and they fit: read once instead of once per tile.
        const int tiles_wg = (tiles + p.NG - 1) / p.NG * (k.pair ? 2 : 1);
        const int lrec_lds = dec8_lds(h.nblk, JG, true).total;
        p.lrec = tiles_wg >= dec8_lrec_min_tiles() && lrec_lds <= kLdsMax &&
                 h.nblk_pad * 32 <= kRecCopy * kDecWaves * 64;
        p.lds = p.lrec ? lrec_lds : dec8_lds(h.nblk, JG).total;
        p.stream = stream_loads(h, k, p, kP8, tiles);
    } else if (dec) {
        p.route = kRouteDec;
        p.quant = fused ? kQuantNone : kQuantStaged;
        p.rs = rs;
        p.lds = lds;
        p.RG = (M + rs - 1) / rs;
        if (p.RG == 1) {
            p.NG = std::min(tiles, n_cu);
        } else {
            p.NG = std::min(tiles, std::max(1, n_cu / p.RG));
            p.pair_xcd = p.NG % 8 == 0 ? 1 : 0;
        }
        p.grid_x = p.NG * p.RG;
        p.flow = flow_phases(h, k, p, tiles);
        p.stream = stream_loads(h, k, p, kProducers, tiles);
    } else {
        p.route = kRouteRows;
        p.quant = kQuantStaged;
        p.grid_x = tiles;
        p.grid_y = (M + kRowsPerWG - 1) / kRowsPerWG;
    }
    return p;
}

// Quantize + block dots + epilogue for M rows on `st`.  Exactly one of
// dC / dCs is non-null; dIdx (optional) receives the per-row argmax.
constexpr int kNotPairable = -100;  // run() with h2: the decode kernel does not take this call

// Handles one decode launch can stream together: the same device and
// device layout; the gate/up pairing also needs the same N.
bool same_layout_but_n(const Handle* a, const Handle* b) {
    return a->device == b->device && a->K == b->K && a->bits == b->bits && a->nbg == b->nbg &&
           a->sc_shift == b->sc_shift && a->ngrp == b->ngrp && a->sc_blk == b->sc_blk && a->extra == b->extra &&
           (a->Z == nullptr) == (b->Z == nullptr) && (a->D == nullptr) == (b->D == nullptr);
}
bool same_layout(const Handle* a, const Handle* b) { return a->N == b->N && same_layout_but_n(a, b); }

// Projections of one activation in one decode launch (i4_matmul_multi_dev).
struct Multi {
    const Handle* h[kMaxSeg];
    float* C[kMaxSeg];
    int n;
    // RMSNorm of the activation in the launch's prologue (the activation
    // holds the rows before the norm).
    bool norm = false;
    const float* normW = nullptr;
    float* normOut = nullptr;
    float eps = 0.0f;
};

// h2 (gate/up pairing): a second handle with the same layout (same_layout).
// Returns kNotPairable, having launched nothing, when the decode kernel does
// not take the call.
// The caller holds w.mu; s is the scratch of st.
// mp (multi-projection): h is mp->h[0] and dC is mp->C[0]; returns
// kNotPairable, having launched nothing, unless one decode launch takes all.
int run(Workspace& w, Scratch& s, Handle* h, const float* dA, int M, float* dC, int32_t* dCs, int64_t* dIdx,
        hipStream_t st, const Handle* h2 = nullptr, const Multi* mp = nullptr) {
    if (M < 0) {
        set_err("M must be >= 0 (got %d)", M);
        return -2;
    }
    if (M == 0) return 0;
    if (!dA || (!dC && !dCs)) {
        set_err("null device pointer");
        return -2;
    }
    if ((reinterpret_cast<uintptr_t>(dA) & 15) != 0) {
        set_err("activations must be 16-byte aligned");
        return -2;
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != h->device) {
        set_err("handle lives on device %d but device %d is current", h->device, dev);
        return -3;
    }
    if ((size_t)M * h->nblk4 > (size_t)std::numeric_limits<int>::max() / 64) {
        set_err("M*K too large");
        return -2;
    }
    const bool hp = g_hi_prec != 0;
    const bool dots = dCs != nullptr;

    GemvArgs a{};
    fill_args(h, a, M);
    a.A = dA;
    a.C = dC;
    a.Cs = dCs;

    CallKind kind;
    kind.dots = dots;
    kind.argmax = dIdx != nullptr;
    kind.pair = h2 != nullptr;
    kind.multi = mp != nullptr;
    kind.norm = mp && mp->norm;
    kind.tiles = a.ntiles;
    if (mp) {
        kind.tiles = 0;
        for (int k = 0; k < mp->n; ++k) kind.tiles += mp->h[k]->N / 16;
    }
    const Plan p = plan_call(shape_of(h), M, kind, device_cus(w, dev));
    if (p.route == kRouteNone) return kNotPairable;

    // The stand-alone quantizer ahead of the matmul kernel.
    if (p.quant == kQuantPrefill) {
        // Records in MFMA operand order for the prefill GEMM.
        const int nch_rec = (h->nblk + 1) / 2;  // record chunks of two blocks
        if (!grow(w, st, &s.rec, &s.rec_cap, (size_t)(p.Mpad / 16) * nch_rec * kRecBytes, "workspace alloc", s.fixed))
            return -4;
        const size_t threads = (size_t)(p.Mpad / 16) * nch_rec * 2 * 64;  // a wave per (16 rows, block)
        const unsigned qb = (unsigned)((threads + 255) / 256);
        if (hp) quantize_rec_kernel<true><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, nch_rec, p.Mpad, s.rec);
        else quantize_rec_kernel<false><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, nch_rec, p.Mpad, s.rec);
        if (!hip_ok(hipGetLastError(), "quantize launch")) return -5;
    } else if (p.quant == kQuantRows8) {
        const int rows8 = dec8_rows(M);
        if (!ensure_quant(w, s, st, rows8, h->nblk4)) return -4;
        const size_t threads = (size_t)rows8 * h->nblk_pad * 4;
        const unsigned qb = (unsigned)((threads + 255) / 256);
        const int JGq = h->bits == 8 ? 2 : 4;
        const int K = h->K, nb = h->nblk, np = h->nblk_pad, n4 = h->nblk4;
        if (hp && JGq == 4)
            quantize_r8_kernel<true, 4><<<qb, 256, 0, st>>>(dA, M, K, nb, np, n4, rows8, s.aq, s.sa, s.sq);
        else if (hp)
            quantize_r8_kernel<true, 2><<<qb, 256, 0, st>>>(dA, M, K, nb, np, n4, rows8, s.aq, s.sa, s.sq);
        else if (JGq == 4)
            quantize_r8_kernel<false, 4><<<qb, 256, 0, st>>>(dA, M, K, nb, np, n4, rows8, s.aq, s.sa, s.sq);
        else
            quantize_r8_kernel<false, 2><<<qb, 256, 0, st>>>(dA, M, K, nb, np, n4, rows8, s.aq, s.sa, s.sq);
        if (!hip_ok(hipGetLastError(), "quantize launch")) return -5;
        a.Aq = s.aq;
        a.Sa = s.sa;
        a.Sq = s.sq;
    } else if (p.quant == kQuantStaged) {
        if (!ensure_quant(w, s, st, M, h->nblk4)) return -4;
        const size_t threads = (size_t)M * h->nblk * 4;
        const unsigned qb = (unsigned)((threads + 255) / 256);
        if (hp) quantize_kernel<true><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, h->nblk4, s.aq, s.sa, s.sq);
        else quantize_kernel<false><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, h->nblk4, s.aq, s.sa, s.sq);
        if (!hip_ok(hipGetLastError(), "quantize launch")) return -5;
        a.Aq = s.aq;
        a.Sa = s.sa;
        a.Sq = s.sq;
    }

    hipError_t e;
    if (mp) {
        int t = 0;
        for (int k = 0; k < kMaxSeg; ++k) {
            if (k < mp->n) {
                a.segW[k] = mp->h[k]->W;
                a.segS[k] = mp->h[k]->S;
                a.segC[k] = mp->C[k];
                a.segN[k] = mp->h[k]->N;
                t += mp->h[k]->N / 16;
                a.seg_end[k] = t;
            } else {
                a.segW[k] = nullptr;
                a.segS[k] = nullptr;
                a.segC[k] = nullptr;
                a.segN[k] = 0;
                a.seg_end[k] = std::numeric_limits<int>::max();
            }
        }
        a.ntiles = t;
        a.normW = mp->normW;
        a.normOut = mp->normOut;
        a.norm_eps = mp->eps;
        const char* ex = std::getenv("BREEZE_HIP_NORM_EXACT");
        a.norm_exact = ex && ex[0] == '1';
    }
    const bool pair = h2 != nullptr;
    if (pair) {
        a.W2 = h2->W;
        a.S2 = h2->S;
        a.Z2 = h2->Z;
        a.D2 = h2->D;
    }
    const int fz = p.split ? kFuseSplit
                   : pair  ? (p.flow ? (p.stream ? kFusePairFlowStream : kFusePairFlow) : kFusePair)
                   : mp    ? (mp->norm ? kFuseNormMulti : kFuseMulti)
                   : p.flow   ? (p.stream ? kFuseFlowStream : kFuseFlow)
                   : p.stream ? kFuseStream
                              : kFusePlain;
    const bool decode = p.route == kRouteDec || p.route == kRouteDec8;
    if (p.split) {
        // Split-K scratch: a ticket per tile (zero between calls; the
        // folding workgroup re-arms it) and each tile's block values.
        const size_t nt = (size_t)a.ntiles, nf = nt * M * 17 * h->nblk4;
        if (s.fixed) {
            // Carved from the call's record region (a split call stages no
            // records); the region holds other data between calls, so a
            // kernel clears the tickets every time.
            const size_t tb = (nt * sizeof(unsigned int) + 255) / 256 * 256;
            if (tb + nf * sizeof(float) > s.rec_cap) {
                set_err("no-allocation scratch: split-K over %zu tiles needs %zu bytes, more than %zu", nt,
                        tb + nf * sizeof(float), s.rec_cap);
                return -4;
            }
            a.stick = reinterpret_cast<unsigned int*>(s.rec);
            a.sf = reinterpret_cast<float*>(s.rec + tb);
            fill_u32_kernel<<<(unsigned)((nt + 63) / 64), 64, 0, st>>>(a.stick, (int)nt, 0u);
            if (!hip_ok(hipGetLastError(), "split ticket clear")) return -5;
        } else {
            const unsigned int* before = s.stick;
            if (!grow(w, st, &s.stick, &s.stick_cap, nt, "split-K workspace") ||
                !grow(w, st, &s.sf, &s.sf_cap, nf, "split-K workspace"))
                return -4;
            if (s.stick != before) {
                // Zeroed once per allocation, on st (a non-blocking stream
                // does not wait for the null stream).
                fill_u32_kernel<<<(unsigned)((s.stick_cap + 63) / 64), 64, 0, st>>>(s.stick, (int)s.stick_cap, 0u);
                if (!hip_ok(hipGetLastError(), "split ticket clear")) return -5;
            }
            a.stick = s.stick;
            a.sf = s.sf;
        }
        a.split = p.split;
    }
    // The decode kernels' in-kernel argmax merges into per-stream state
    // (a ticket, then kDecMaxRows row keys), zero between calls.
    if (decode && dIdx) {
        if (!s.ticket && s.fixed) {
            set_err("internal: fixed scratch without argmax state");
            return -5;
        }
        if (!s.ticket) {
            // Allocated and zeroed once per stream, outside capture; the
            // kernel's last workgroup re-arms it to zero.
            if (capturing(st)) {
                set_err("argmax workspace: make one argmax call on the stream before capturing it");
                return -4;
            }
            unsigned int* t = nullptr;
            if (!hip_ok(hipMalloc(&t, (1 + kDecMaxRows) * sizeof(unsigned long long)), "argmax workspace"))
                return -4;
            // Cleared on st itself: a non-blocking stream does not wait
            // for work on the null stream.
            fill_u32_kernel<<<(2 * (1 + kDecMaxRows) + 63) / 64, 64, 0, st>>>(t, 2 * (1 + kDecMaxRows), 0u);
            if (!hip_ok(hipGetLastError(), "argmax workspace clear")) {
                w.retired.push_back(t);
                return -4;
            }
            s.ticket = t;
        }
        a.ticket = s.ticket;
        a.key = reinterpret_cast<unsigned long long*>(s.ticket) + 1;
        a.idx = dIdx;
    }
    if (decode) {
        a.RS = p.rs;
        a.RG = p.RG;
        a.NG = p.NG;
        a.pair_xcd = p.pair_xcd;
    }
    const bool x = h->extra;
    if (p.route == kRouteDec8) {
        const uint4* rec = reinterpret_cast<const uint4*>(s.aq);
        bool* at = &w.dec8_attr[16 * ((h->bits == 8 ? 1 : 0) | (hp ? 2 : 0))];
        if (h->bits == 8) e = hp ? launch_dec8<8, true>(at, a, rec, p.grid_x, p.lds, fz, x, p.lrec, st)
                                 : launch_dec8<8, false>(at, a, rec, p.grid_x, p.lds, fz, x, p.lrec, st);
        else e = hp ? launch_dec8<4, true>(at, a, rec, p.grid_x, p.lds, fz, x, p.lrec, st)
                    : launch_dec8<4, false>(at, a, rec, p.grid_x, p.lds, fz, x, p.lrec, st);
    } else if (p.route == kRouteDec) {
        const bool fu = p.fused, p64 = p.p64;
        if (h->bits == 8) e = hp ? launch_dec_bits<8, true>(w.attr_set, a, p.grid_x, p.lds, fz, p64, fu, x, st)
                                 : launch_dec_bits<8, false>(w.attr_set, a, p.grid_x, p.lds, fz, p64, fu, x, st);
        else e = hp ? launch_dec_bits<4, true>(w.attr_set, a, p.grid_x, p.lds, fz, p64, fu, x, st)
                    : launch_dec_bits<4, false>(w.attr_set, a, p.grid_x, p.lds, fz, p64, fu, x, st);
    } else if (p.route == kRoutePrefill) {
        PfArgs pa{};
        pa.W = reinterpret_cast<const char*>(h->W);
        pa.WS = reinterpret_cast<const char*>(h->WS);
        pa.S = reinterpret_cast<const char*>(h->S);
        pa.Z = reinterpret_cast<const char*>(h->Z);
        pa.R = reinterpret_cast<const char*>(s.rec);
        pa.C = dC;
        pa.M = M;
        pa.N = h->N;
        pa.nblk = h->nblk;
        pa.nch = (h->nblk + 1) / 2;
        pa.ngrp = h->ngrp;
        pa.sc_shift = h->sc_shift;
        pa.ntiles = h->N / 16;
        pa.nbg = h->nbg;
        const int scm = h->sc_blk ? 2 : (h->sc_shift == 31 ? 0 : 1);
        if (h->bits == 4 && scm == 2 && !h->Z) {
            set_err("internal: INT4 handle with per-block scales has no zero points");
            return -5;
        }
        const dim3 grid((unsigned)p.grid_x, (unsigned)p.grid_y);
        if (h->bits == 8)
            e = hp ? launch_pf<8, true>(w.pf_attr, pa, scm, p.pf_rp, p.pf_ct, grid, st)
                   : launch_pf<8, false>(w.pf_attr, pa, scm, p.pf_rp, p.pf_ct, grid, st);
        else
            e = hp ? launch_pf<4, true>(w.pf_attr, pa, scm, p.pf_rp, p.pf_ct, grid, st)
                   : launch_pf<4, false>(w.pf_attr, pa, scm, p.pf_rp, p.pf_ct, grid, st);
    } else {
        const dim3 grid((unsigned)p.grid_x, (unsigned)p.grid_y);
        if (h->bits == 8) e = hp ? launch_rows_bits<8, true>(a, grid, dots, st)
                                 : launch_rows_bits<8, false>(a, grid, dots, st);
        else e = hp ? launch_rows_bits<4, true>(a, grid, dots, st) : launch_rows_bits<4, false>(a, grid, dots, st);
    }
    if (!hip_ok(e, "matmul launch")) return -5;

    if (dIdx && !dots && !decode) {
        // Both decode kernels merge their own argmax (last workgroup).
        const int nparts = (h->N + kArgmaxChunk - 1) / kArgmaxChunk;
        if (!grow(w, st, &s.parts, &s.parts_cap, (size_t)M * nparts, "argmax workspace", s.fixed)) return -4;
        argmax_partial_kernel<<<dim3(nparts, M), 256, 0, st>>>(dC, h->N, s.parts);
        argmax_final_kernel<<<M, 256, 0, st>>>(s.parts, nparts, M, dIdx);
        if (!hip_ok(hipGetLastError(), "argmax launch")) return -5;
    }
    return 0;
}

// Runs f(w, s) on the current device with its lock held and the scratch of
// stream st.  Every device entry point that launches matmul work goes
// through here, so calls from several host threads serialize per device.
template <typename F>
int with_scratch(const Handle* h, hipStream_t st, F&& f) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != h->device) {
        set_err("handle lives on device %d but device %d is current", h->device, dev);
        return -3;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_err("device ordinal %d out of range", dev);
        return -3;
    }
    Workspace& w = g_ws[dev];
    std::lock_guard<std::mutex> lock(w.mu);
    Scratch* s = scratch_for(w, st);
    if (!s) return -4;
    return f(w, *s);
}

// The decoder's RMSNorm on device pointers (i4_rmsnorm_dev), on stream st.
int launch_rmsnorm(const float* dX, const float* dW, int M, int H, float eps, float* dOut, hipStream_t st) {
    if (M < 0 || H <= 0) {
        set_err("need M >= 0 and H > 0 (got M %d, H %d)", M, H);
        return -1;
    }
    if (M == 0) return 0;
    if (!dX || !dW || !dOut) {
        set_err("null device pointer");
        return -2;
    }
    // BREEZE_HIP_NORM_EXACT=1 always takes the in-order reconstruction (tests).
    const char* ex = std::getenv("BREEZE_HIP_NORM_EXACT");
    const int exact_only = ex && ex[0] == '1';
    if (H <= kNormStage)
        rmsnorm_kernel<true><<<(unsigned)M, kNormThreads, (size_t)H * sizeof(float), st>>>(dX, dW, H, eps, dOut,
                                                                                           exact_only);
    else
        rmsnorm_kernel<false><<<(unsigned)M, kNormThreads, 0, st>>>(dX, dW, H, eps, dOut, exact_only);
    return hip_ok(hipGetLastError(), "rmsnorm launch") ? 0 : -3;
}

bool check_dims(int N, int K, int bits) {
    if (N <= 0 || K <= 0 || N % 16 || K % 32 || (bits != 4 && bits != 8)) {
        set_err("contract violation: need N>0, K>0, N%%16==0, K%%32==0, bits in {4,8} "
                "(got N=%d K=%d bits=%d)", N, K, bits);
        return false;
    }
    // The decode kernels address a handle's weights with 32-bit cursors in
    // 16-byte chunks: at most 2^32 chunks (64 GiB of packed weights).
    const uint64_t jg = bits == 8 ? 2 : 4;
    const uint64_t chunks = (uint64_t)(N / 16) * ((uint64_t)(K / 32) + jg - 1) / jg * 64;
    if (chunks > 0xFFFFFFFFull) {
        set_err("weights of N=%d K=%d at %d bits take %llu 16-byte chunks; the kernels address at most 2^32 "
                "(64 GiB)", N, K, bits, (unsigned long long)chunks);
        return false;
    }
    return true;
}

}  // namespace

// ====================================================================== C ABI

extern "C" {

void i4_set_threads(int) {}
void i4_set_numa_split(int) {}
void i4_set_hi_prec(int on) { g_hi_prec = on; }

const char* i4_last_error(void) { return g_err.c_str(); }

int i4_device_ok(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        set_err("no HIP device");
        return 0;
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        set_err("hipGetDeviceProperties failed");
        return 0;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_err("device %d is %s; this library is built for gfx950", dev, prop.gcnArchName);
        return 0;
    }
    hipFuncAttributes attr;
    if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&quantize_kernel<true>)) !=
        hipSuccess) {
        set_err("gfx950 kernels not loadable");
        return 0;
    }
    return 1;
}

void* i4_prepack_onnx(const uint8_t* qw, const void* scales, const uint8_t* qzeros, int N, int K,
                      int bits, int scale_bits) {
    if (!qw || !scales) {
        set_err("null weights or scales");
        return nullptr;
    }
    if (scale_bits != 16 && scale_bits != 32) {
        set_err("scale_bits must be 16 or 32 (got %d)", scale_bits);
        return nullptr;
    }
    if (bits == 8 && qzeros) {
        set_err("INT8 weights take no zero points (symmetric 128)");
        return nullptr;
    }
    if (!check_dims(N, K, bits)) return nullptr;
    const int nblk = K / 32;
    if ((size_t)N > (std::numeric_limits<size_t>::max() - 63) / (size_t)nblk / (size_t)(4 * bits)) {
        set_err("size overflow");
        return nullptr;
    }
    const size_t blocks = (size_t)N * nblk;
    std::vector<float> sc(blocks);
    if (scale_bits == 16) {
        const uint8_t* s = static_cast<const uint8_t*>(scales);
        for (size_t i = 0; i < blocks; ++i) {
            uint16_t x;
            std::memcpy(&x, s + 2 * i, 2);
            sc[i] = half_to_float(x);
        }
    } else {
        std::memcpy(sc.data(), scales, blocks * 4);
    }
    std::vector<int8_t> zp;
    if (bits == 4 && qzeros) {
        zp.resize(blocks);
        bool all8 = true;
        const int packed = (nblk + 1) / 2;
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < nblk; ++j) {
                const int z = (qzeros[(size_t)n * packed + j / 2] >> (4 * (j % 2))) & 15;
                zp[(size_t)n * nblk + j] = (int8_t)z;
                all8 = all8 && z == 8;
            }
        if (all8) zp.clear();
    }
    return build_handle(qw, false, sc.data(), N, K, bits, zp, {});
}

void* i4_prepack(const uint8_t* B, const float* scale, const int8_t* zp, const int32_t* corr, int N,
                 int K, int nblk, int bits) {
    if (!B || !scale || !corr || (bits == 4 && !zp)) {
        set_err("null legacy input");
        return nullptr;
    }
    if (!check_dims(N, K, bits)) return nullptr;
    if (nblk != K / 32) {
        set_err("nblk must equal K/32");
        return nullptr;
    }
    const int ntiles = N / 16, gbytes = bits == 8 ? 64 : 32;
    const size_t blocks = (size_t)N * nblk;
    // Unpack the pre-transformed layout to signed weights b[n][k], exactly as
    // the reference tile kernels read it (unpack_kgroup, _mm512_sub_epi8).
    std::vector<int8_t> b((size_t)N * K);
    std::vector<int8_t> nib;
    std::vector<int8_t> zpv;
    std::vector<float> sc(blocks);
    std::vector<int32_t> delta(blocks);
    bool zp_fits = true;
    if (bits == 4) {
        nib.resize((size_t)N * K);
        zpv.resize(blocks);
    }
    for (int t = 0; t < ntiles; ++t)
        for (int j = 0; j < nblk; ++j) {
            const size_t meta = ((size_t)t * nblk + j) * 16;
            const uint8_t* blk = B + ((size_t)t * nblk + j) * 8 * gbytes;
            for (int col = 0; col < 16; ++col) {
                const int n = t * 16 + col;
                int32_t sum = 0;
                for (int g = 0; g < 8; ++g)
                    for (int k = 0; k < 4; ++k) {
                        const int v = col * 4 + k;
                        int val;
                        if (bits == 8) {
                            val = (int8_t)blk[g * 64 + v];
                        } else {
                            const uint8_t byte = blk[g * 32 + v / 2];
                            const int x = (v & 1) ? byte >> 4 : byte & 15;
                            nib[(size_t)n * K + 32 * j + g * 4 + k] = (int8_t)x;
                            val = (int8_t)(uint8_t)(x - zp[meta + col]);
                        }
                        b[(size_t)n * K + 32 * j + g * 4 + k] = (int8_t)val;
                        sum += val;
                    }
                sc[(size_t)n * nblk + j] = scale[meta + col];
                delta[(size_t)n * nblk + j] = 128 * sum - corr[meta + col];
                if (bits == 4) {
                    zpv[(size_t)n * nblk + j] = zp[meta + col];
                    zp_fits = zp_fits && zp[meta + col] >= -112;
                }
            }
        }
    bool any_delta = false;
    for (int32_t d : delta) any_delta = any_delta || d != 0;
    if (!any_delta) delta.clear();
    if (bits == 8 || !zp_fits) {
        // Signed bytes [N][nblk][32]; INT4 with zero points below -112 would
        // wrap in int8 arithmetic, so such handles keep the wrapped values.
        return build_handle(reinterpret_cast<const uint8_t*>(b.data()), true, sc.data(), N, K, 8, {}, delta);
    }
    std::vector<uint8_t> raw(blocks * 16);
    for (size_t n = 0; n < (size_t)N; ++n)
        for (int i = 0; i < K / 2; ++i)
            raw[n * (K / 2) + i] = (uint8_t)((nib[n * K + 2 * i] & 15) | (nib[n * K + 2 * i + 1] & 15) << 4);
    bool all8 = true;
    for (int8_t z : zpv) all8 = all8 && z == 8;
    if (all8) zpv.clear();
    return build_handle(raw.data(), false, sc.data(), N, K, 4, zpv, delta);
}

void i4_free(void* handle) {
    if (!handle) return;
    Handle* h = as_handle(handle);
    if (!h) return;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(h->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(h->W);
    (void)hipFree(h->S);
    if (h->Z) (void)hipFree(h->Z);
    if (h->D) (void)hipFree(h->D);
    if (h->WS) (void)hipFree(h->WS);
    (void)hipSetDevice(cur);
    h->magic = 0;
    delete h;
}

int i4_matmul_dev(void* handle, const float* dA, int M, float* dC, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    return with_scratch(h, st, [&](Workspace& w, Scratch& s) { return run(w, s, h, dA, M, dC, nullptr, nullptr, st); });
}

int i4_matmul_silu_mul_dev(void* gate, void* up, const float* dA, int M, float* dC, void* stream) {
    Handle* hg = as_handle(gate);
    Handle* hu = as_handle(up);
    if (!hg || !hu) return -1;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (hg->N != hu->N || hg->K != hu->K) {
        set_err("gate and up projections differ in shape (N %d/%d, K %d/%d)", hg->N, hu->N, hg->K, hu->K);
        return -2;
    }
    if (hg->device != hu->device) {
        set_err("gate and up projections live on devices %d and %d", hg->device, hu->device);
        return -3;
    }
    return with_scratch(hg, st, [&](Workspace& w, Scratch& s) {
        if (same_layout(hg, hu)) {
            const int rc = run(w, s, hg, dA, M, dC, nullptr, nullptr, st, hu);
            if (rc != kNotPairable) return rc;
        }
        // Two projections, then the elementwise epilogue.
        if (M <= 0 || !dC) return run(w, s, hu, dA, M, dC, nullptr, nullptr, st);
        const size_t n = (size_t)M * hg->N;
        if (!grow(w, st, &s.gate, &s.gate_cap, n, "workspace alloc")) return -4;
        int rc = run(w, s, hg, dA, M, s.gate, nullptr, nullptr, st);
        if (rc == 0) rc = run(w, s, hu, dA, M, dC, nullptr, nullptr, st);
        if (rc) return rc;
        silu_mul_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(s.gate, dC, dC, n);
        return hip_ok(hipGetLastError(), "silu-mul launch") ? 0 : -5;
    });
}

int i4_silu_mul_dev(const float* dG, const float* dU, size_t n, float* dOut, void* stream) {
    if (n == 0) return 0;
    if (!dG || !dU || !dOut) {
        set_err("null device pointer");
        return -2;
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t blocks = (n + 255) / 256;
    if (blocks > 0x7FFFFFFFu) {
        set_err("silu-mul: %zu elements are more than one launch covers", n);
        return -2;
    }
    silu_mul_kernel<<<(unsigned)blocks, 256, 0, st>>>(dG, dU, dOut, n);
    return hip_ok(hipGetLastError(), "silu-mul launch") ? 0 : -5;
}

int i4_matmul_multi_dev(void* const* handles, int n, const float* dA, int M, float* const* dC, void* stream) {
    if (!handles || !dC || n < 1 || n > kMaxSeg) {
        set_err("need 1 to %d handles and as many outputs (got %d)", kMaxSeg, n);
        return -2;
    }
    Multi mp{};
    mp.n = n;
    for (int i = 0; i < n; ++i) {
        Handle* h = as_handle(handles[i]);
        if (!h) return -1;
        if (!dC[i]) {
            set_err("null device pointer");
            return -2;
        }
        if (i > 0 && (h->K != mp.h[0]->K || h->device != mp.h[0]->device)) {
            set_err("projections of one activation need one K and one device");
            return -2;
        }
        mp.h[i] = h;
        mp.C[i] = dC[i];
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    Handle* h0 = const_cast<Handle*>(mp.h[0]);
    return with_scratch(h0, st, [&](Workspace& w, Scratch& s) {
        bool one = n > 1;
        for (int i = 1; i < n; ++i) one = one && same_layout_but_n(h0, mp.h[i]);
        if (one) {
            const int rc = run(w, s, h0, dA, M, mp.C[0], nullptr, nullptr, st, nullptr, &mp);
            if (rc != kNotPairable) return rc;
        }
        for (int i = 0; i < n; ++i) {
            const int rc = run(w, s, const_cast<Handle*>(mp.h[i]), dA, M, mp.C[i], nullptr, nullptr, st);
            if (rc) return rc;
        }
        return 0;
    });
}

int i4_matmul_argmax_dev(void* handle, const float* dA, int M, float* dC, int64_t* dIdx, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    if (!dIdx) {
        set_err("null argmax output");
        return -2;
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    return with_scratch(h, st, [&](Workspace& w, Scratch& s) { return run(w, s, h, dA, M, dC, nullptr, dIdx, st); });
}

int i4_matmul_noalloc_dev(void* handle, const float* dA, int M, float* dC, int64_t* dIdx, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    if (M < 0) {
        set_err("M must be >= 0 (got %d)", M);
        return -2;
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != h->device) {
        set_err("handle lives on device %d but device %d is current", h->device, dev);
        return -3;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_err("device ordinal %d out of range", dev);
        return -3;
    }
    Workspace& w = g_ws[dev];
    std::lock_guard<std::mutex> lock(w.mu);
    if (!g_noalloc_ptr[dev]) {
        void* p = nullptr;
        if (!hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "no-allocation scratch address")) return -4;
        g_noalloc_ptr[dev] = static_cast<uint8_t*>(p);
    }
    uint8_t* base = g_noalloc_ptr[dev];
    // Argmax partials at the end (they follow the matmul launch, so their
    // room is set aside first), activation records in between.
    const size_t nparts = dIdx ? (size_t)M * ((h->N + kArgmaxChunk - 1) / kArgmaxChunk) : 0;
    const size_t parts_bytes = (nparts * sizeof(unsigned long long) + 255) / 256 * 256;
    if (kNoAllocState + parts_bytes > kNoAllocBytes) {
        set_err("no-allocation scratch: %d rows of argmax partials need %zu bytes, more than %zu", M, parts_bytes,
                kNoAllocBytes - kNoAllocState);
        return -4;
    }
    const size_t region = kNoAllocBytes - kNoAllocState - parts_bytes;
    Scratch s{};
    s.fixed = true;
    s.stream = st;
    s.ticket = reinterpret_cast<unsigned int*>(base);
    s.parts = reinterpret_cast<unsigned long long*>(base + kNoAllocBytes - parts_bytes);
    s.parts_cap = parts_bytes / sizeof(unsigned long long);
    uint8_t* recs = base + kNoAllocState;
    s.rec = recs;
    s.rec_cap = region;
    // Stand-alone quantizer records for this call's rows: [M][nblk4] of 64 B
    // records, then the scales and sums.
    const size_t nq = (size_t)(M >= 5 && M <= kDec8MaxRows ? dec8_rows(M) : M) * h->nblk4;
    if (nq * 72 <= region) {
        s.aq = recs;
        s.sa = reinterpret_cast<float*>(recs + nq * 64);
        s.sq = reinterpret_cast<int*>(recs + nq * 68);
        s.aq_cap = nq * 64;
        s.sa_cap = s.sq_cap = nq;
    }
    if (dIdx && M > 0) {
        // The decode argmax merges into this state and needs it zero; a
        // kernel clears it (a graph may capture this call).
        fill_u32_kernel<<<(2 * (1 + kDecMaxRows) + 63) / 64, 64, 0, st>>>(s.ticket, 2 * (1 + kDecMaxRows), 0u);
        if (!hip_ok(hipGetLastError(), "argmax state clear")) return -5;
    }
    return run(w, s, h, dA, M, dC, nullptr, dIdx, st);
}

int i4_block_dots_dev(void* handle, const float* dA, int M, int32_t* dCs, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    return with_scratch(h, st, [&](Workspace& w, Scratch& s) { return run(w, s, h, dA, M, nullptr, dCs, nullptr, st); });
}

void i4_matmul(void* handle, const float* A, int M, float* C) {
    g_err.clear();
    Handle* h = as_handle(handle);
    if (!h) return;
    if (M <= 0) {
        if (M < 0) set_err("M must be >= 0 (got %d)", M);
        return;
    }
    if (!A || !C) {
        set_err("null host pointer");
        return;
    }
    int cur = 0;
    (void)hipGetDevice(&cur);
    if (cur != h->device && !hip_ok(hipSetDevice(h->device), "set device")) return;
    struct Restore {
        int cur, dev;
        ~Restore() {
            if (cur != dev) (void)hipSetDevice(cur);
        }
    } restore{cur, h->device};
    Workspace& w = g_ws[h->device];
    std::lock_guard<std::mutex> lock(w.mu);
    if (!w.stream && !hip_ok(hipStreamCreateWithFlags(&w.stream, hipStreamNonBlocking), "stream")) return;
    Scratch* s = scratch_for(w, w.stream);
    if (!s) return;
    const size_t na = (size_t)M * h->K, nc = (size_t)M * h->N;
    if (!grow(w, w.stream, &w.hA, &w.hA_cap, na, "staging alloc") ||
        !grow(w, w.stream, &w.hC, &w.hC_cap, nc, "staging alloc"))
        return;
    if (!hip_ok(hipMemcpyAsync(w.hA, A, na * 4, hipMemcpyHostToDevice, w.stream), "upload A")) return;
    if (run(w, *s, h, w.hA, M, w.hC, nullptr, nullptr, w.stream) != 0) {
        (void)hipStreamSynchronize(w.stream);
        return;
    }
    if (!hip_ok(hipMemcpyAsync(C, w.hC, nc * 4, hipMemcpyDeviceToHost, w.stream), "download C")) return;
    (void)hip_ok(hipStreamSynchronize(w.stream), "matmul");
}

void i4_matmul_region(void* handle, const float* A, int M, float* C, uint8_t*, float*) {
    i4_matmul(handle, A, M, C);
}

int i4_plan_query(int bits, int M, int K, int N, int flags, int n_cu, int32_t* out, int nout) {
    if (!out || nout < 1 || M < 1 || n_cu < 1) {
        set_err("plan query: needs out, nout >= 1, M >= 1 and n_cu >= 1");
        return -1;
    }
    if (!check_dims(N, K, bits)) return -1;
    const int JG = bits == 8 ? 2 : 4;
    Shape h{};
    h.bits = bits;
    h.N = N;
    h.nblk = K / 32;
    h.nblk4 = (h.nblk + 3) / 4 * 4;
    h.nblk_pad = (h.nblk + JG - 1) / JG * JG;
    h.extra = (flags & 32) != 0 || (flags & 64) != 0;
    h.has_dl = (flags & 64) != 0;
    h.has_ws = bits == 8;  // every INT8 handle carries its weight sums
    CallKind k;
    k.dots = (flags & 1) != 0;
    k.argmax = (flags & 2) != 0;
    k.pair = (flags & 4) != 0;
    k.multi = (flags & 8) != 0;
    k.norm = (flags & 16) != 0;
    k.tiles = N / 16;
    const Plan p = plan_call(h, M, k, n_cu);
    const int32_t v[] = {p.route, p.quant, p.fused, p.p64, p.lrec, p.rs, p.RG, p.NG, p.pair_xcd, p.lds,
                         p.pf_rp, p.pf_ct, p.grid_x, p.grid_y, p.split, p.stream, p.flow};
    const int n = std::min(nout, (int)(sizeof(v) / sizeof(v[0])));
    for (int i = 0; i < n; ++i) out[i] = v[i];
    return n;
}

int i4_handle_info(void* handle, int64_t* out) {
    Handle* h = as_handle(handle);
    if (!h || !out) return -1;
    out[0] = h->N;
    out[1] = h->K;
    out[2] = h->bits;
    out[3] = h->sc_group;
    out[4] = h->has_zp;
    out[5] = h->has_dl;
    out[6] = (int64_t)h->dev_bytes;
    out[7] = h->device;
    return 0;
}

int i4_unpack(void* handle, uint8_t* qw, float* scales, uint8_t* zp, int32_t* corr_delta) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    const int N = h->N, nblk = h->nblk, bits = h->bits;
    const size_t blocks = (size_t)N * nblk;
    if (qw) {
        std::vector<uint4> W((size_t)(N / 16) * h->nbg * 64);
        if (!hip_ok(hipMemcpy(W.data(), h->W, W.size() * 16, hipMemcpyDeviceToHost), "download")) return -5;
        const int JG = bits == 8 ? 2 : 4;
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < nblk; ++j)
                for (int oct = 0; oct < 4; ++oct) {
                    const int t = n / 16, lane = oct * 16 + (n % 16), cg = j / JG, jb = j % JG;
                    const uint4 v = W[((size_t)t * h->nbg + cg) * 64 + lane];
                    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
                    if (bits == 8) {
                        uint8_t* dst = qw + ((size_t)n * nblk + j) * 32 + oct * 8;
                        for (int p = 0; p < 4; ++p) dst[p] = (uint8_t)((words[2 * jb] >> (8 * p)) ^ 0x80u);
                        for (int p = 0; p < 4; ++p) dst[4 + p] = (uint8_t)((words[2 * jb + 1] >> (8 * p)) ^ 0x80u);
                    } else {
                        uint8_t* dst = qw + ((size_t)n * nblk + j) * 16 + oct * 4;
                        uint8_t nibs[8];
                        for (int b = 0; b < 4; ++b) {
                            const uint8_t t8 = (uint8_t)(words[jb] >> (8 * b));
                            nibs[b] = t8 & 15;
                            nibs[4 + b] = t8 >> 4;
                        }
                        for (int i = 0; i < 4; ++i) dst[i] = (uint8_t)(nibs[2 * i] | nibs[2 * i + 1] << 4);
                    }
                }
    }
    if (scales) {
        const size_t cnt = h->sc_blk ? (size_t)N * h->nblk_pad : (size_t)N * h->ngrp;
        std::vector<float> S(cnt);
        if (!hip_ok(hipMemcpy(S.data(), h->S, cnt * 4, hipMemcpyDeviceToHost), "download")) return -5;
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < nblk; ++j)
                scales[(size_t)n * nblk + j] = h->sc_blk ? S[blk_index(n, j, h->nbg, bits == 8 ? 2 : 4)]
                                                         : S[grp_index(n, j, h->ngrp, h->sc_shift)];
    }
    if (zp) {
        if (h->Z && h->bits == 4) {
            std::vector<int8_t> Z((size_t)N * h->nblk4);
            if (!hip_ok(hipMemcpy(Z.data(), h->Z, Z.size(), hipMemcpyDeviceToHost), "download")) return -5;
            for (int n = 0; n < N; ++n)
                for (int j = 0; j < nblk; ++j) zp[(size_t)n * nblk + j] = (uint8_t)Z[blk_index(n, j, h->nbg, 4)];
        } else {
            std::memset(zp, bits == 8 ? 128 : 8, blocks);
        }
    }
    if (corr_delta) {
        if (h->D) {
            std::vector<int32_t> Dv((size_t)N * h->nblk_pad);
            if (!hip_ok(hipMemcpy(Dv.data(), h->D, Dv.size() * 4, hipMemcpyDeviceToHost), "download")) return -5;
            for (int n = 0; n < N; ++n)
                for (int j = 0; j < nblk; ++j)
                    corr_delta[(size_t)n * nblk + j] = Dv[blk_index(n, j, h->nbg, bits == 8 ? 2 : 4)];
        } else {
            std::memset(corr_delta, 0, blocks * 4);
        }
    }
    return 0;
}

int i4_rmsnorm_dev(const float* dX, const float* dW, int M, int H, float eps, float* dOut, void* stream) {
    return launch_rmsnorm(dX, dW, M, H, eps, dOut, static_cast<hipStream_t>(stream));
}

int i4_rmsnorm_matmul_multi_dev(const float* dX, const float* dNormW, float eps, void* const* handles, int n, int M,
                                float* const* dC, float* dHn, void* stream) {
    if (!handles || !dC || n < 1 || n > kMaxSeg) {
        set_err("need 1 to %d handles and as many outputs (got %d)", kMaxSeg, n);
        return -2;
    }
    if (!dX || !dNormW) {
        set_err("null device pointer");
        return -2;
    }
    Multi mp{};
    mp.n = n;
    for (int i = 0; i < n; ++i) {
        Handle* h = as_handle(handles[i]);
        if (!h) return -1;
        if (!dC[i]) {
            set_err("null device pointer");
            return -2;
        }
        if (i > 0 && (h->K != mp.h[0]->K || h->device != mp.h[0]->device)) {
            set_err("projections of one activation need one K and one device");
            return -2;
        }
        mp.h[i] = h;
        mp.C[i] = dC[i];
    }
    mp.norm = true;
    mp.normW = dNormW;
    mp.normOut = dHn;
    mp.eps = eps;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    Handle* h0 = const_cast<Handle*>(mp.h[0]);
    const int K = h0->K;
    return with_scratch(h0, st, [&](Workspace& w, Scratch& s) {
        bool one = true;
        for (int i = 1; i < n; ++i) one = one && same_layout_but_n(h0, mp.h[i]);
        if (one && M > 0) {
            const int rc = run(w, s, h0, dX, M, mp.C[0], nullptr, nullptr, st, nullptr, &mp);
            if (rc != kNotPairable) return rc;
        }
        if (M <= 0) return M < 0 ? run(w, s, h0, dX, M, mp.C[0], nullptr, nullptr, st) : 0;
        // The norm as its own launch, then the projections.
        float* hn = dHn;
        if (!hn) {
            if (!grow(w, st, &s.hn, &s.hn_cap, (size_t)M * K, "workspace alloc")) return -4;
            hn = s.hn;
        }
        int rc = launch_rmsnorm(dX, dNormW, M, K, eps, hn, st);
        if (rc) return rc;
        Multi plain = mp;
        plain.norm = false;
        if (one) {
            rc = run(w, s, h0, hn, M, plain.C[0], nullptr, nullptr, st, nullptr, &plain);
            if (rc != kNotPairable) return rc;
        }
        for (int i = 0; i < n; ++i) {
            rc = run(w, s, const_cast<Handle*>(mp.h[i]), hn, M, mp.C[i], nullptr, nullptr, st);
            if (rc) return rc;
        }
        return 0;
    });
}

}  // extern "C"

// qmm_common.h -- what the translation units of libbreeze_qmm.so share: the
// handle and its device layout, the device helpers (quantizer, operand
// unpacking, MFMA wrappers), the decode and prefill kernels' argument
// structs and LDS layouts, and the launchers each kernel unit exports.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

typedef int v4i __attribute__((ext_vector_type(4)));

namespace bq {

// ------------------------------------------------------------------ layout

// Device weight layout: chunk (t, c) of 16-column tile t is 64 lanes x 16
// bytes; lane l serves column 16t + (l & 15) and k-octet (l >> 4) of each
// block -- the B operand of v_mfma_i32_16x16x32_i8, in natural k order.
//   INT8: 2 blocks per chunk, 8 signed bytes (raw ^ 0x80) per block.
//   INT4: 4 blocks per chunk, one dword per block whose byte b holds the
//         nibbles of k = 8*octet + b (low) and k = 8*octet + 4 + b (high), so
//         `w & 0x0F0F0F0F` and `(w >> 4) & 0x0F0F0F0F` are k 0..3 and 4..7.
// Activation record per (row, block): 64 bytes, part 0 then part 1, each 32
// bytes in natural k order: INT16 mode h then l (signed halves), INT8 mode q
// then zeros.

constexpr uint32_t kMagic = 0xB2EE2E51u;
constexpr int kFlagZp = 1, kFlagDl = 2, kFlagScBlk = 4;

struct Handle {
    uint32_t magic;
    int N, K, nblk, bits;  // bits of the device representation
    int nbg;               // 16-byte chunks per tile along K
    int nblk_pad;          // nbg * blocks per chunk
    int nblk4;             // nblk rounded up to 4
    int sc_shift, ngrp, sc_group;
    bool sc_blk;           // scales stored per block [N][nblk_pad]
    bool has_zp, has_dl;   // explicit zero points / legacy corr supplied
    bool extra;            // per-block scale, zp (INT4) and corr arrays materialized
    int device;
    uint4* W;    // [N/16][nbg][64] 16-byte chunks
    float* S;    // [N][ngrp], or [N][nblk_pad] when sc_blk
    int8_t* Z;   // [N][nblk4] zero points (INT4 extra handles only)
    int32_t* D;  // [N][nblk_pad] legacy corr delta (extra handles only)
    int32_t* WS; // INT8 handles: 128 * per-block weight sums, [N/16][nbg][16][2]
    size_t dev_bytes;
};

// Per-column metadata is tile-major, so the 16 columns a lane group reads
// for one chunk are contiguous:
//   scales (per column or per group of 2^sc_shift blocks): [N/16][ngrp][16];
//   per-block arrays of EXTRA handles, JG blocks per chunk:
//     scales, corr delta: [N/16][nbg][16][JG]; INT4 zero points: [N/16][nbg][16][4] bytes.
__host__ __device__ inline size_t grp_index(int n, int j, int ngrp, int sc_shift) {
    return ((size_t)(n >> 4) * ngrp + (j >> sc_shift)) * 16 + (n & 15);
}
__host__ __device__ inline size_t blk_index(int n, int j, int nbg, int JG) {
    return (((size_t)(n >> 4) * nbg + j / JG) * 16 + (n & 15)) * JG + j % JG;
}

// ------------------------------------------------------------------ device helpers

__device__ inline int dpp_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
__device__ inline int dpp_xor2(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false); }

// Quantizes one 32-block (quantize_A / quantize_A_i16 of one block,
// kernel/quantized_matmul.cpp:215-258) with 4 lanes, 8 consecutive k per
// lane (lane q of the quad holds k = 8q..8q+7).  Returns the block scale
// and sum(q) in every lane of the quad, and this lane's 8 bytes of record
// part 0 (ph: the INT8 values, or the high bytes in the two-pass mode) and
// part 1 (pl: the low bytes).  All 64 lanes of the wave must call it.
template <bool HP>
__device__ inline void quant4x8(float4 v0, float4 v1, float& s_out, uint2& ph, uint2& pl, int& sum_out) {
    const float x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    // amax over the block from +0 with NaNs skipped, as the reference's
    // `a > amax ? a : amax` does.  fmaxf returns the other operand of a quiet
    // NaN; canonicalizing first makes every NaN quiet, and the +0 operand
    // keeps a lane whose values are all NaN at 0.
    float ab[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ab[i] = fabsf(__builtin_canonicalizef(x[i]));
    float amax = fmaxf(fmaxf(fmaxf(fmaxf(ab[0], ab[1]), 0.0f), fmaxf(ab[2], ab[3])),
                       fmaxf(fmaxf(ab[4], ab[5]), fmaxf(ab[6], ab[7])));
    int am = __float_as_int(amax);  // >= +0: integer order is float order
    am = max(am, dpp_xor1(am));
    am = max(am, dpp_xor2(am));
    amax = __int_as_float(am);
    constexpr int qmax = HP ? 32767 : 127;
    // s = amax / qmax, correctly rounded: the product with fl(1 / qmax) and
    // one FMA correction, which equals the IEEE quotient for every finite
    // amax >= +0 (checked exhaustively against division for both qmax;
    // the subnormals included).  amax = inf keeps the quotient inf.
    constexpr float kInvQ = 1.0f / (float)qmax;
    const float q0 = amax * kInvQ;
    const float s = __builtin_isinf(amax) ? amax : __builtin_fmaf(__builtin_fmaf(-q0, (float)qmax, amax), kInvQ, q0);
    float inv = s > 0.0f ? 1.0f / s : 0.0f;
    // The reference gives q = 0 for a non-finite product (its lrint).  An
    // infinite inv (a block scale too small for its reciprocal) makes every
    // product of the block infinite or NaN, so inv = 0 gives the same
    // zeros.  With inv finite, the only non-finite products are NaN (a NaN
    // element, or an infinite one times inv = 1 / inf = 0), and
    // v_cvt_i32_f32 converts NaN to 0.  The reference's clamp to +-qmax
    // never binds when inv is finite: |x| <= amax, and rint(amax * inv) <=
    // qmax for every finite amax (checked exhaustively for both qmax).
    if (__builtin_isinf(inv)) inv = 0.0f;
    int q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // Hardware conversion (NaN -> 0), which C's conversion does not promise.
        asm("v_cvt_i32_f32 %0, %1" : "=v"(q[i]) : "v"(__builtin_rintf(x[i] * inv)));
    }
    int sum = (q[0] + q[1] + q[2]) + (q[3] + q[4] + q[5]) + (q[6] + q[7]);
    // Bytes by v_perm_b32 (selector byte k picks byte k of the second
    // operand for 0-3, of the first for 4-7).  q as 16-bit two's complement
    // is u - 32768 for u = q + 32768, so its high byte is the reference's
    // (u >> 8) - 128 and its low byte (u & 255) - 128 after flipping bit 7.
    uint32_t w0[2], w1[2] = {0u, 0u};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t* qq = reinterpret_cast<const uint32_t*>(q + 4 * h);
        if (HP) {
            const uint32_t p01 = __builtin_amdgcn_perm(qq[1], qq[0], 0x05040100u);  // q1.lo16 : q0.lo16
            const uint32_t p23 = __builtin_amdgcn_perm(qq[3], qq[2], 0x05040100u);
            w0[h] = __builtin_amdgcn_perm(p23, p01, 0x07050301u);                 // high bytes
            w1[h] = __builtin_amdgcn_perm(p23, p01, 0x06040200u) ^ 0x80808080u;   // low bytes
        } else {
            const uint32_t p01 = __builtin_amdgcn_perm(qq[1], qq[0], 0x05040400u);  // q1.b0 : q0.b0 in bytes 0-1
            const uint32_t p23 = __builtin_amdgcn_perm(qq[3], qq[2], 0x05040400u);
            w0[h] = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
        }
    }
    s_out = s;
    ph = make_uint2(w0[0], w0[1]);
    pl = make_uint2(w1[0], w1[1]);
    sum += dpp_xor1(sum);
    sum_out = sum + dpp_xor2(sum);
}
template <bool HP>
__device__ inline void quant4x8(float4 v0, float4 v1, float& s_out, uint2& ph, uint2& pl) {
    int sum;
    quant4x8<HP>(v0, v1, s_out, ph, pl, sum);
}

__device__ inline uint64_t unpack_b(const uint4& w, int jb, int bits) {
    if (bits == 8) {
        const uint32_t lo = jb == 0 ? w.x : w.z, hi = jb == 0 ? w.y : w.w;
        return (uint64_t)hi << 32 | lo;
    }
    const uint32_t x = jb == 0 ? w.x : jb == 1 ? w.y : jb == 2 ? w.z : w.w;
    return (uint64_t)((x >> 4) & 0x0F0F0F0Fu) << 32 | (x & 0x0F0F0F0Fu);
}

__device__ inline v4i mfma16(uint64_t a, uint64_t b) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, v4i{0, 0, 0, 0}, 0, 0, 0);
}

// v_mfma_i32_16x16x64_i8: A byte i of lane l multiplies B byte i of lane
// (column + 16 * (l >> 4)), so a lane's first 8 bytes pair with the first
// block of a decode chunk's block pair and its last 8 bytes with the second
// (the decode parity tests with one and two rows pin this pairing: any other
// would change the exact block sums).
// v_mfma_i32_32x32x32_i8 (full INT8 rate, one 32-block of k): A byte i of
// lane l is row l & 31, k 16 * (l >> 5) + i; B byte i of lane l is k
// 16 * (l >> 5) + i, column l & 31; result j of lane l is row
// (j & 3) + 8 * (j >> 2) + 4 * (l >> 5), column l & 31.
typedef int v16i __attribute__((ext_vector_type(16)));
__device__ inline v16i mfma32(const v4i& a, const v4i& b, const v16i& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ inline v4i mfma64(const uint4& a, const uint4& b) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i{(int)a.x, (int)a.y, (int)a.z, (int)a.w},
                                                   v4i{(int)b.x, (int)b.y, (int)b.z, (int)b.w},
                                                   v4i{0, 0, 0, 0}, 0, 0, 0);
}


// ------------------------------------------------------------------ decode GEMV (up to 16 rows)
//
// One workgroup of 16 waves per CU owns a contiguous range of 16-column
// tiles for up to 4 activation rows (5 to 16 rows: one workgroup per row
// group of 4, the row groups of a tile range placed on the same XCD so the
// later reads of every weight chunk hit its L2).  Waves 0..14 produce: a tile's K range is cut into
// phases of 15 chunks and producer w takes chunk 15p + w of phase p, so
// every producer streams its weights in K order and the chunks of a phase
// arrive together.  Per phase each producer runs the MFMA and the in-lane
// epilogue of its chunk and writes f = f32(cs) * scale to an LDS phase
// buffer.  Wave 15 loads no weights: after each phase's workgroup barrier
// it folds that phase's blocks in order, acc = fma(s, f, acc), while the
// producers work on the next phase (two phase buffers), and it writes C at
// each tile end.  The phase buffer holds each output lane's f values
// contiguously, so the fold of a full phase is wide LDS reads and one FMA
// per block.
//
// Weight chunks are loaded R units ahead through a register ring; the first
// R units go out at kernel start, behind only the activation loads, and
// stream in while the activations are quantized into LDS (FUSED) or their
// records, made by the stand-alone quantizer, are copied there.  Every load
// is unconditional (units past the end re-read the last tile) and the ring is
// unrolled, so the compiler's load waits stay exact across the loop back
// edge.

constexpr int kDecWaves = 16;
constexpr int kChainWave = kDecWaves - 1;
constexpr int kProducers = kDecWaves - 1;
// The quantizing prologue (4 lanes per 32-block, quant4x8) runs on the first
// eight waves when one pass of 128 blocks covers the activations: the last
// waves of a workgroup start up to ~0.3 us after the first, and the prologue
// barrier waits for the slowest quantizer.  More blocks take all sixteen
// waves (at most kQuantPasses passes of 256).
constexpr int kQuantEarlyBlocks = 128, kQuantPasses = 6;
// Most row-blocks a launch with the RMSNorm in its prologue takes (two
// quantize passes), and so the longest lane run of block sums per row.
constexpr int kNormFusedMaxBlocks = 3 * 128;
constexpr int kNormRun = (kNormFusedMaxBlocks + 63) / 64;

struct GemvArgs {
    const uint4* W;
    const float* S;
    const int8_t* Z;
    const int32_t* D;
    const float* A;        // fp32 [M][K]
    const uint8_t* Aq;     // [M][nblk][64] records (stand-alone quantizer)
    const float* Sa;       // [M][nblk4]
    const int* Sq;         // [M][nblk4]
    float* C;              // [M][N]
    int32_t* Cs;           // [M][N][nblk] (block-dot export)
    int64_t* idx;              // [M] argmax, or NULL
    unsigned int* ticket;      // with idx: workgroups done (0 between calls)
    unsigned long long* key;   // with idx: [8] merged argmax keys (0 between calls)
    // Second weight set for the gate/up pairing, in the same layout as W, S,
    // Z, D (same N, K, bits and scale grouping).
    const uint4* W2;
    const float* S2;
    const int8_t* Z2;
    const int32_t* D2;
    int M, N, K, nblk, nblk4, nbg, nblk_pad, sc_shift, ngrp, flags;
    int ntiles, NG, RG, pair_xcd;
    int RS;  // rows per row group: 4, or 2 or 1 where four rows of records do not fit
    // Multi-projection launch: up to kMaxSeg weight sets of one layout (all
    // but N alike) whose 16-column tiles are concatenated in order; segment
    // k owns tiles [seg_end[k - 1], seg_end[k]) and writes segC[k], a
    // [M][segN[k]] array.  Unused entries have seg_end = INT_MAX.
    const uint4* segW[4];
    const float* segS[4];
    float* segC[4];
    int segN[4];
    int seg_end[4];
    // RMSNorm in the prologue (kFuseNormMulti): A holds the rows before the
    // norm; normW [K] its weights, normOut [M][K] (or NULL) receives the
    // normalized rows.
    const float* normW;
    float* normOut;
    float norm_eps;
    int norm_exact;  // always take the in-order sum (tests)
    // Split-K (kFuseSplit): split workgroups per tile; sf receives each
    // tile's per-block values and activation scales ([tile][M][17][nblk4]
    // floats: columns 0..15, then the scales), stick counts the workgroups
    // of each tile that are done (0 between calls).
    float* sf;
    unsigned int* stick;
    int split;
};
constexpr int kMaxSeg = 4;

// Decode kernel modes: one weight set, the gate/up pair with the SiLU
// epilogue, several projections of one activation, the same with the
// decoder's RMSNorm applied to the activation in the prologue, one weight
// set split along K (each workgroup takes a range of one tile's phases; the
// last to finish folds the tile), and one weight set whose chunks are read
// with non-temporal loads (kFuseStream: the plain kernel otherwise).
// kFuseFlow and kFuseFlowStream are the plain kernel (with ordinary or
// non-temporal loads) whose phases run across tile boundaries: the chunks
// of a workgroup's tiles form one stream, so a tile's short last phase is
// filled with the next tile's first chunks.
// kFusePairFlow and kFusePairFlowStream do the same for the gate/up pair,
// whose stream alternates a column tile's gate and up chunks.
constexpr int kFusePlain = 0, kFusePair = 1, kFuseMulti = 2, kFuseNormMulti = 3, kFuseSplit = 4, kFuseStream = 5,
              kFuseFlow = 6, kFuseFlowStream = 7, kFusePairFlow = 8, kFusePairFlowStream = 9;

// One weight chunk of a wave plus its per-column metadata.  EXTRA handles
// (explicit zero points, legacy corr, scale groups smaller than a chunk)
// carry materialized per-block arrays so every load is unconditional.
// Eight consecutive activation floats of one lane (k = 8q..8q+7 of a block).
struct Oct {
    uint4 x, y;
};

template <int JG, bool EXTRA>
struct Unit {
    uint4 w;
    float sc[EXTRA ? JG : 1];
    int dl[EXTRA ? JG : 1];
    uint32_t zp;  // INT4 zero points, one byte per block
    int c;        // chunk to compute; nbg or more: none (past the end)
};

// ------------------------------------------------------------------ SiLU
//
// The reference's siluf (kernel/qwen35_decoder.cpp:128) is x / (1 + std::exp(-x))
// in float, and std::exp(float) there is the host C library's expf: glibc's
// table-driven expf (since glibc 2.27; x86-64 runs its FMA build), which is
// not correctly rounded.  ref_expf restates that published method step for
// step, in double: x * 32/ln2 = k + r with k = round(x * 32/ln2) and r from
// fused multiply-adds, exp(x) = 2^(k/32) * (1 + c2 r + c1 r^2 + c0 r^3), the
// 2^(i/32) factors (correctly rounded to double, exponent field offset by
// -i/32) from a table, one rounding to float at the end; below and above the
// range the library's own overflow and underflow results.  Equal to the host
// expf on every float (the tests compare them exhaustively), so the fused
// SiLU matches the reference bit for bit.
__host__ __device__ inline float ref_expf(float x) {
    static constexpr uint64_t kTab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
    constexpr double kInvLn2N = 0x1.71547652b82fep+5;  // 32 / ln 2
    constexpr double kShift = 0x1.8p+52;               // rounds to an integer in the low bits
    constexpr double kC0 = 0x1.c6af84b912394p-20, kC1 = 0x1.ebfce50fac4f3p-13, kC2 = 0x1.62e42ff0c52d6p-6;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    if (((ux >> 20) & 0x7ff) >= 0x42b) {  // |x| >= 88, inf or NaN
        if (ux == 0xff800000u) return 0.0f;
        if (((ux >> 20) & 0x7ff) >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();  // exp(x) above the float range
        if (x < -0x1.9fe368p6f) return 0.0f;              // below half the smallest subnormal
    }
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const double s = __builtin_bit_cast(double, kTab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(kC0, r, kC1);
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r * r, y);
    return (float)(y * s);
}

// silu(g) * u exactly as the reference's loop (qwen35_decoder.cpp:408) forms it.
__host__ __device__ inline float silu_mul(float g, float u) { return g / (1.0f + ref_expf(-g)) * u; }

__device__ inline unsigned long long argmax_key(float v, int idx) {
    uint32_t o;
    if (v != v) {
        o = 0xFFFFFFFFu;
    } else if (v == 0.0f) {
        o = 0x80000000u;
    } else {
        const uint32_t b = __float_as_uint(v);
        o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return (unsigned long long)o << 32 | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}

// RMSNorm's mean (float)(ss / H) from a tree sum T of the squares (all
// >= 0, each exact): every term passes through at most D = per + 22
// roundings of the tree, so |T - S| <= gamma_D * S for the exact sum S, and
// the reference's in-order double sum ss (kernel/qwen35_decoder.cpp:137)
// satisfies |ss - S| <= gamma_(H-1) * S; ss lies within E = (H + D + 2) *
// 2^-53 * T (with slack for gamma and for rounding T -/+ E) of T.
// S -> (float)(S / H) is monotone, so when T - E and T + E map to the same
// float, that is (float)(ss / H).  Returns whether the bound decided it.
__device__ inline bool norm_mean_from_bound(double T, int H, int per, float* mean) {
    const double E = (double)(H + per + 24) * 0x1p-53 * T * (1.0 + 0x1p-10);
    const float lo = (float)((T - E) / (double)H), hi = (float)((T + E) / (double)H);
    *mean = lo;
    return lo == hi;
}

// The same decision with rH = RN(1 / H) in place of the two divisions (rH
// can be formed before T is known).  With u = 2^-53 and Q = T / H,
// q = RN(T rH) is within 2.01 u Q of Q, so ss / H lies within
// E / H + 2.01 u Q of q.  D = (E rH + 2^-50 q)(1 + 2^-10) exceeds that by at
// least 1.98 u q, more than the rounding of q -/+ D, so RN(q - D) and
// RN(q + D) bracket every ss / H, and (float) of both agreeing decides it as
// above.  T must be finite and >= 0; a sum of float squares is 0 or
// >= 2^-298, far above double underflow, so the relative bounds hold.
__device__ inline bool norm_mean_from_bound_r(double T, int H, double rH, int per, float* mean) {
    const double E = (double)(H + per + 24) * 0x1p-53 * T * (1.0 + 0x1p-10);
    const double q = T * rH;
    const double D = (E * rH + q * 0x1p-50) * (1.0 + 0x1p-10);
    const float lo = (float)(q - D), hi = (float)(q + D);
    *mean = lo;
    return lo == hi;
}

// Sum of a double over the four 16-lane rows of a wave, the same in every
// lane: rows (0 + 2) and (1 + 3) by a half swap, then those two by a row
// swap (two roundings a term).
__device__ inline double sum_rows_f64(double v) {
    auto swap_add = [](double x, bool half) {
        const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
        const unsigned lo = (unsigned)b, hi = (unsigned)(b >> 32);
        const auto l = half ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                            : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
        const auto h = half ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                            : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
        const double a = __builtin_bit_cast(double, (unsigned long long)h[0] << 32 | l[0]);
        const double c = __builtin_bit_cast(double, (unsigned long long)h[1] << 32 | l[1]);
        return a + c;
    };
    return swap_add(swap_add(v, true), false);
}

__device__ inline long long readlane64(long long v, int l) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)v, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)((unsigned long long)v >> 32), l);
    return (long long)((unsigned long long)hi << 32 | lo);
}

// Sums of doubles over lane groups by DPP (no LDS permutes): every lane of
// each aligned 8-lane octet, or 16-lane row, gets its group's sum, each term
// passing through 3 or 4 roundings.
__device__ inline double dpp_f64(double v, int ctrl) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    int lo = (int)(unsigned)b, hi = (int)(unsigned)(b >> 32);
    switch (ctrl) {  // the control must be a constant
        case 0xB1:
            lo = __builtin_amdgcn_update_dpp(0, lo, 0xB1, 0xF, 0xF, false);
            hi = __builtin_amdgcn_update_dpp(0, hi, 0xB1, 0xF, 0xF, false);
            break;
        case 0x4E:
            lo = __builtin_amdgcn_update_dpp(0, lo, 0x4E, 0xF, 0xF, false);
            hi = __builtin_amdgcn_update_dpp(0, hi, 0x4E, 0xF, 0xF, false);
            break;
        case 0x141:
            lo = __builtin_amdgcn_update_dpp(0, lo, 0x141, 0xF, 0xF, false);
            hi = __builtin_amdgcn_update_dpp(0, hi, 0x141, 0xF, 0xF, false);
            break;
        default:
            lo = __builtin_amdgcn_update_dpp(0, lo, 0x140, 0xF, 0xF, false);
            hi = __builtin_amdgcn_update_dpp(0, hi, 0x140, 0xF, 0xF, false);
            break;
    }
    return __builtin_bit_cast(double, (unsigned long long)(unsigned)hi << 32 | (unsigned)lo);
}
__device__ inline double sum8_f64(double v) {
    v += dpp_f64(v, 0xB1);         // lane ^ 1
    v += dpp_f64(v, 0x4E);         // lane ^ 2
    return v + dpp_f64(v, 0x141);  // 7 - lane within the octet
}
__device__ inline double sum16_f64(double v) {
    v = sum8_f64(v);
    return v + dpp_f64(v, 0x140);  // 15 - lane within the row
}

// The reference's in-order double sum of squares of x[0..H), by one wave
// (every lane returns it): the slow way, for rows the bound does not decide.
// UNROLL: lane reads unrolled per 64-element step.  Fully unrolled (64) the
// stand-alone norm kernel's fallback takes 42 us a row of 5120, unrolled by
// 8 it takes 110 us; but fully unrolled inside the decode kernel the 128
// lane reads were hoisted into scalar registers and spilled (239 SGPRs),
// so the decode kernel's prologue, where this is a rare path, unrolls by 8.
template <int UNROLL>
__device__ inline double norm_sumsq_inorder(const float* x, int H) {
    // Every lane of the wave holds the same running sum; the wave squares 64
    // elements at a time (exactly, in double) and each term enters the sum
    // in element order through v_readlane, so only the adds form the chain.
    const int lane = threadIdx.x & 63;
    double ss = 0.0;
    int c = 0;
    for (; c + 64 <= H; c += 64) {
        const float v = x[c + lane];
        const long long tb = __builtin_bit_cast(long long, (double)v * (double)v);
#pragma unroll UNROLL
        for (int l = 0; l < 64; ++l) ss += __builtin_bit_cast(double, readlane64(tb, l));
    }
    if (c < H) {
        const float v = c + lane < H ? x[c + lane] : 0.0f;
        const long long tb = __builtin_bit_cast(long long, (double)v * (double)v);
        for (int l = 0; l < H - c; ++l) ss += __builtin_bit_cast(double, readlane64(tb, l));
    }
    return ss;
}

// Barrier that orders LDS only: outstanding global loads stay in flight.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// f row pitch (floats) of the phase buffer: 15 chunks of JG blocks plus
// padding that keeps the JG-wide stores and reads free of bank conflicts.
__host__ __device__ constexpr int dec_pitch(int JG) { return kProducers * JG + (JG == 4 ? 8 : 4); }

// LDS layout of the decode kernel for Mr_max activation rows per workgroup.
// The host sizes the launch with it and the kernel rebuilds it from its
// preloaded arguments.  With more than one row the row pitches are padded
// so the rows read by one lane group fall on different banks: records 64 B
// past a multiple of 256 B, block scales and sums 16 B past one.
struct DecLds {
    int rec_pitch;  // bytes per activation row of records
    int sa_pitch;   // elements per row of block scales / sums
    int recs, sa, sq, consts, fbuf, total;  // byte offsets, bytes used
};

__host__ __device__ inline int lds_take(int& off, int bytes) {
    const int o = off;
    off += (bytes + 15) / 16 * 16;
    return o;
}

// P64 (one or two rows, block pairs per MFMA): each 8-byte k-octet of a
// record sits in a 16-byte slot behind 8 zero bytes, 128 B per block plus
// one zero slot at the row end, so one 16-byte read yields [octet | zeros]
// or [zeros | octet]; the row pitch of the second row is 32 B past a
// multiple of 256 B.
__host__ __device__ inline DecLds dec_lds(int Mr_max, int nblk, int JG, bool p64 = false) {
    DecLds l;
    // The 16x16x32 layout stores whole chunks ([h, l][k-octet][block]), so a
    // row spans every chunk, padding blocks included.
    l.rec_pitch = p64 ? nblk * 128 + 16 : (nblk + JG - 1) / JG * JG * 64;
    l.sa_pitch = (nblk + 3) / 4 * 4;
    if (Mr_max > 1) {
        l.rec_pitch = p64 ? (l.rec_pitch + 223) / 256 * 256 + 32 : (l.rec_pitch + 191) / 256 * 256 + 64;
        l.sa_pitch = (l.sa_pitch + 59) / 64 * 64 + 4;
    }
    int off = 0;
    l.recs = lds_take(off, Mr_max * l.rec_pitch);
    l.sa = lds_take(off, Mr_max * l.sa_pitch * 4);
    l.sq = lds_take(off, Mr_max * l.sa_pitch * 4);
    l.consts = lds_take(off, 512);
    l.fbuf = lds_take(off, 2 * 64 * dec_pitch(JG) * 4);
    l.total = off;
    return l;
}

// Split-K block values cross workgroups (and XCDs, whose L2 caches are not
// coherent for ordinary stores) as device-scope atomic stores of JG floats,
// two at a time: written through to the device's coherence point.
template <int JG>
__device__ inline void store_agent(float* dst, const float* src_lds) {
#pragma unroll
    for (int h = 0; h < JG / 2; ++h) {
        const uint2 v = *reinterpret_cast<const uint2*>(src_lds + 2 * h);
        __hip_atomic_store(reinterpret_cast<uint64_t*>(dst) + h, (uint64_t)v.y << 32 | v.x, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Blocks of LDS records (and scales) a split-K workgroup holds: its piece's
// chunks, at most ceil(npw / S) phases of 15 and at most the tile's nbg,
// indexed from the piece's first block.
__host__ __device__ inline int split_piece_blocks(int npw, int S, int nbg, int JG) {
    const int ch = (npw + S - 1) / S * kProducers;
    return (ch < nbg ? ch : nbg) * JG;
}

// Split-K fold staging: the tile's [M][17][nblk4] floats copied to LDS at
// offset 0 (over the records and phase buffers, dead by then) with a row
// pitch of nblk4 + 4 floats, so the 16 columns' rows start 16 B apart in the
// banks; a flag word follows the larger of that and the kernel's layout.
__host__ __device__ inline int split_pitch(int nblk4) { return nblk4 + 4; }
__host__ __device__ inline int split_flag_off(int M, int nblk4, int layout_total) {
    const int stage = M * 17 * split_pitch(nblk4) * 4;
    const int end = stage > layout_total ? stage : layout_total;
    return (end + 15) / 16 * 16;
}

// Ring depth R (weight units in flight per wave).  Two units per producer
// (30 KB per CU) measured fastest on every decode workload: deeper rings
// put more requests in flight than the memory system turns into bandwidth.
constexpr int kDecRing = 2;

constexpr int kLdsMax = 160 * 1024;

// ------------------------------------------------------------------ prefill GEMM (more rows)
//
// One workgroup of 8 waves computes 32 RP rows (RP = 1, 2 or 4 row pairs of
// 16-row tiles) x 16*CT columns over all of K.  Wave w owns row pair w % RP
// and column part w / RP of the 8 / RP parts (CT / parts tiles each, the
// first CT % parts parts one more); waves w and w + 4 share a SIMD.  With
// RP = 4 the parts are two halves: the C4 shape's 512 rows fill the CUs
// with 128-row workgroups, while fewer rows use 32- or 64-row workgroups
// and split the columns over more waves instead of leaving waves without
// rows.  Per 32-block, H = sum(h*b) comes from one MFMA, (H << 8) + 128*S is
// the accumulator input of the l-byte MFMA, which then holds the exact block
// integer cs, and the lane folds acc = fma(s_a, f32(cs) * s_b, acc) in block
// order.  Pairs of tiles run on v_mfma_i32_32x32x32_i8, an odd last tile on
// v_mfma_i32_16x16x32_i8.
//
// Operands reach LDS by direct global->LDS loads (global_load_lds_dwordx4,
// 16 bytes per lane to LDS address M0 + 16*lane) through a ring of S stages
// of two chunks (S = 2, or 3 for the 32- and 64-row shapes, whose short
// stages would not cover a load's latency).  A chunk (two blocks) holds the
// CT weight
// tiles (1 KB each; the decode layout is the MFMA B operand), their weight
// sums and scales (the shared part, loaded by all waves together), and the
// workgroup's 2 RP activation records (also split over all waves).  The
// compiler does not see these loads: every
// wave waits for its own with an explicit vmcnt, then the workgroup barrier
// publishes the stage.
//
// INT4 weights (BITS 4) take the same core.  A stage is one INT4 chunk (four
// blocks, 1 KB per tile), loaded raw into chunk 0's weight area; its scales
// and zero points go to one raw area shared by both stages.  After the
// stage barrier all 512 threads expand it in place: per byte, b = nibble -
// zp as a signed byte (n + (128 - zp)) ^ 0x80, chunk 0 getting blocks 0-1
// and chunk 1 blocks 2-3 in the INT8 chunk layout, plus 128 * sum(b) per
// (column, block) for the two-pass product and the scales in the INT8
// chunk layout.  A second barrier publishes the expanded stage.

constexpr int kPfWaves = 8;
// Chunks per ring stage.
constexpr int kPfChunks = 2;
// Activation record per (16-row tile, chunk): per block 1 KB, h bytes then
// l bytes, each [k half 2][row 16][16 B]: the 16 bytes of (row r, k half kh)
// are k-octets 2 kh and 2 kh + 1 of row r, the v_mfma_i32_32x32x32_i8 A
// operand of lane r + 16 kh (one 16-byte LDS read, no register moves).  Then
// the block scales [block 2][row 16] float.
constexpr int kRecA = 2048, kRecBytes = kRecA + 128;
// Byte of (row r, k-octet o) in a block's h half of a record.
__host__ __device__ constexpr int pf_rec_byte(int r, int o) { return 16 * (r + 16 * (o >> 1)) + 8 * (o & 1); }
// Byte of (column c, k-octet o) of block b in a weight tile's 1 KB in LDS.
// INT8 tiles arrive by DMA in the decode chunk order (octet o of both blocks
// at 16 (c + 16 o)), so a 32x32x32 B operand takes two 8-byte halves.  INT4
// tiles are expanded in LDS into [column half][k half][block][column c & 7]
// [16 B]: one conflict-free 16-byte read per operand.
__host__ __device__ constexpr int pf_w_byte(int bits, int c, int o, int b) {
    return bits == 8 ? 16 * (c + 16 * o) + 8 * b : 16 * ((c & 7) + 8 * b + 16 * (o >> 1) + 32 * (c >> 3)) + 8 * (o & 1);
}

struct PfArgs {
    const char* W;   // INT8: [ntiles][nch][64 lanes][16 B]; INT4: [ntiles][nbg][64][16 B]
    const char* WS;  // INT8: [ntiles][nch][16][2] int32
    const char* S;   // scales (grp_index / blk_index layouts)
    const char* Z;   // INT4 per-block zero points [ntiles][nbg][16][4] (SCM 2 only)
    const char* R;   // activation records [Mpad/16][nch][kRecBytes]
    float* C;        // [M][N]
    int M, N, nblk, nch, ngrp, sc_shift, ntiles;
    int nbg;         // INT4: 4-block chunks per tile
};

// SCM: scale layout: 0 one per column, 1 per group of >= 2 blocks, 2 per block.
// One chunk's LDS region: [CT weight tiles, 1 KB each][weight sums, 128 B
// per tile][block or group scales][2 RP activation records].  INT4 adds kNRaw
// raw areas after the S stages, stage g using area g % kNRaw: S - 1 when a
// barrier follows the expansion (only the next stage waits for its expansion
// while the one after it loads), S with one row pair, whose waves expand
// their own tiles with no barrier after it (a wave may load stage g + S - 1
// while another still expands stage g).  A raw area holds group scales
// (SCM 1, 64 B per tile) or block scales then zero points (SCM 2, 256 + 64 B
// per tile), in whole KB.
template <int CT, int SCM, int BITS, int RP, int S>
struct PfLayout {
    static constexpr int kWS = CT * 1024;
    static constexpr int kSB = kWS + CT * 128;
    static constexpr int kSharedUsed = kSB + (SCM == 2 ? CT * 128 : SCM == 1 ? CT * 64 : 0);
    // INT8 pads the sums and scales to whole KB: their 1 KB loads start
    // where the weight tiles end and must not run into the records.
    static constexpr int kShared = BITS == 8 ? kWS + (kSharedUsed - kWS + 1023) / 1024 * 1024 : kSharedUsed;
    static constexpr int kA = kShared;
    static constexpr int kChunk = kA + 2 * RP * kRecBytes;
    static constexpr int kStage = kPfChunks * kChunk;
    static constexpr int kRawZ = CT * 256;  // SCM 2: zero points after the block scales
    static constexpr int kRawUsed = BITS == 8 ? 0 : SCM == 2 ? CT * 320 : SCM == 1 ? CT * 64 : 0;
    static constexpr int kRaw = (kRawUsed + 1023) / 1024 * 1024;
    static constexpr int kRawOff = S * kStage;  // raw area r at kRawOff + r * kRaw
    static constexpr int kNRaw = RP == 1 ? S : S - 1;
    // INT8, per chunk: CT weight tiles of 1 KB, kWJ a wave; then the sums
    // and scales in kSU units of 1 KB, kSJ a wave.
    static constexpr int kWJ = BITS == 8 ? (CT + kPfWaves - 1) / kPfWaves : 0;
    static constexpr int kSU = BITS == 8 ? (kShared - kWS) / 1024 : 0;
    static constexpr int kSJ = (kSU + kPfWaves - 1) / kPfWaves;
    // INT4, per stage: the CT raw tiles and the raw area in units of 1 KB.
    static constexpr int kUnits = CT + kRaw / 1024;
    // Shared loads a wave issues per chunk (INT8) or stage (INT4).
    static constexpr int kPerWave = BITS == 8 ? kWJ + kSJ : (kUnits + kPfWaves - 1) / kPfWaves;
    static constexpr int kBytes = kRawOff + kNRaw * kRaw;
    static_assert(kShared % 64 == 0 && kBytes <= 160 * 1024, "layout");
};

__device__ inline uint32_t lds_address(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 16 bytes per lane from global `src` to LDS byte address lds + 16*lane.
__device__ inline void dma16(const void* src, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

// The same from a uniform base and a per-lane 32-bit byte offset: the address
// arithmetic stays on the scalar unit.
__device__ inline void dma16s(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// s_waitcnt immediate: vmcnt(n), no wait on the other counters.
__host__ __device__ constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00; }


// Instantiated (row pairs, column tiles) per workgroup.  Every column part
// has at least one tile (CT >= 8 / RP).
struct PfCfg {
    int rp, ct, st;  // row pairs, column tiles, ring stages
};
constexpr PfCfg kPfCfgs[] = {{4, 17, 2}, {4, 16, 2}, {4, 13, 2}, {4, 12, 2}, {4, 9, 2}, {4, 8, 2}, {4, 5, 2},
                             {4, 4, 2},  {2, 16, 2}, {2, 8, 3},  {2, 4, 3},  {1, 16, 2}, {1, 8, 3}};
constexpr int kPfNumCfgs = sizeof(kPfCfgs) / sizeof(kPfCfgs[0]);

// ------------------------------------------------------------------ decode in row groups of eight
//
// dec8_kernel (dec8_kernel.h): 14 producer waves (chunk 14p + w of phase p)
// and two chain waves per workgroup of eight activation rows.
constexpr int kP8 = 14;
constexpr int kRows8 = 8;

// LDS: block scales and (INT4) -zp * sum(q) of the eight rows, row pitch
// padded 16 B past a multiple of 256 B (the four rows a fold or epilogue
// reads together fall on different banks), then the phase buffer
// [2 buffers][2 rows][64 lanes][dec8_pitch(JG)] of f values, then (LREC) the
// row group's activation records in their global layout.
// Phase-buffer pitch (floats per lane) for 14 producers: JG-wide stores
// and reads at this lane stride fall on distinct banks (60 l mod 64 are
// distinct multiples of 4 over 16 lanes; 34 as in dec_kernel for JG = 2).
__host__ __device__ constexpr int dec8_pitch(int JG) { return JG == 4 ? 60 : dec_pitch(JG); }
static_assert(kP8 * 4 <= 60, "a producer's slot in the phase buffer");

struct Dec8Lds {
    int sa_pitch;         // elements per row
    int sa, sq, fbuf, recs, total;  // byte offsets, bytes used
};
__host__ __device__ inline Dec8Lds dec8_lds(int nblk, int JG, bool lrec = false) {
    Dec8Lds l;
    l.sa_pitch = ((nblk + 3) / 4 * 4 + 59) / 64 * 64 + 4;
    int off = 0;
    l.sa = lds_take(off, kRows8 * l.sa_pitch * 4);
    l.sq = lds_take(off, kRows8 * l.sa_pitch * 4);
    l.fbuf = lds_take(off, 2 * 2 * 64 * dec8_pitch(JG) * 4);
    l.recs = lds_take(off, lrec ? (nblk + JG - 1) / JG * JG * 512 : 0);
    l.total = off;
    return l;
}
// Records copied into LDS (LREC): at most this many uint4 per thread.
constexpr int kRecCopy = 8;

// Launchers, one explicit instantiation per (bits, activation mode) in the
// kernel units dec_w*.hip and pf_w*.hip.  attr_set / pf_attr: this device's
// flags of kernels whose dynamic LDS limit is already raised.
template <int BITS, bool HP>
hipError_t launch_dec_bits(bool* attr_set, const GemvArgs& a, int grid, int lds, int fuse, bool p64, bool fused,
                           bool extra, hipStream_t st);
// The five-to-eight-row decode kernel (dec8_kernel.h): rec holds the
// activation records in MFMA operand order, written by quantize_r8_kernel.
template <int BITS, bool HP>
hipError_t launch_dec8(bool* attr_set, const GemvArgs& a, const uint4* rec, int grid, int lds, int fuse, bool extra,
                       bool lrec, hipStream_t st);
template <int BITS, bool HP>
hipError_t launch_pf(bool* pf_attr, const PfArgs& p, int scm, int rp, int ct, dim3 grid, hipStream_t st);

}  // namespace bq

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

typedef int v4i __attribute__((ext_vector_type(4)));

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

Handle* as_handle(void* p) {
    auto* h = static_cast<Handle*>(p);
    if (!h || h->magic != kMagic) {
        set_err("invalid handle");
        return nullptr;
    }
    return h;
}

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
__device__ inline int dpp_mirror8(int v) { return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false); }

// max over the 8 lanes of an aligned lane octet.  Inputs are +0 or more and
// never NaN, so their bit patterns order as the floats do.
__device__ inline float max8(float xf) {
    int x = __float_as_int(xf);
    x = max(x, dpp_xor1(x));
    x = max(x, dpp_xor2(x));
    return __int_as_float(max(x, dpp_mirror8(x)));
}

__device__ inline int sum8(int x) {
    x += dpp_xor1(x);
    x += dpp_xor2(x);
    return x + dpp_mirror8(x);
}

// Quantizes one 32-block with 8 lanes, 4 consecutive k per lane (lane e of
// the octet holds k = 4e..4e+3).  All 64 lanes of the wave must call it.
// Returns the block scale and sum(q) in every lane of the octet, and this
// lane's 4 bytes of record part 0 and part 1.
template <bool HP>
__device__ inline void quant8(float4 v, float& s_out, int& sum_out, uint32_t& p0, uint32_t& p1) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    // amax over the block from +0 with NaNs skipped, as the reference's
    // `a > amax ? a : amax` does.  fmaxf returns the other operand of a quiet
    // NaN; canonicalizing first makes every NaN quiet, and the +0 operand
    // keeps a lane whose values are all NaN at 0.
    const float a0 = fabsf(__builtin_canonicalizef(x[0])), a1 = fabsf(__builtin_canonicalizef(x[1]));
    const float a2 = fabsf(__builtin_canonicalizef(x[2])), a3 = fabsf(__builtin_canonicalizef(x[3]));
    float amax = fmaxf(fmaxf(fmaxf(a0, a1), 0.0f), fmaxf(a2, a3));
    amax = max8(amax);
    constexpr int qmax = HP ? 32767 : 127;
    const float s = amax / (float)qmax;
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    int sum = 0;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float prod = x[i] * inv;
        int q = 0;
        if (__builtin_isfinite(prod)) {
            q = (int)rintf(prod);
            q = q > qmax ? qmax : (q < -qmax ? -qmax : q);
        }
        sum += q;
        if (HP) {
            const uint32_t u = (uint32_t)(q + 32768);
            w0 |= (((u >> 8) ^ 0x80u) & 0xFFu) << (8 * i);
            w1 |= (((u & 0xFFu) ^ 0x80u) & 0xFFu) << (8 * i);
        } else {
            w0 |= ((uint32_t)q & 0xFFu) << (8 * i);
        }
    }
    s_out = s;
    sum_out = sum8(sum);
    p0 = w0;
    p1 = w1;
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

// Stand-alone activation quantizer: 8 lanes per (row, block).  Records go
// to Aq [M][nblk][64 B]; scale and sum(q) to Sa/Sq [M][nblk4].
template <bool HP>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ A, int M, int K,
                                                       int nblk, int nblk4, uint8_t* __restrict__ Aq,
                                                       float* __restrict__ Sa, int* __restrict__ Sq) {
    const int gtid = blockIdx.x * 256 + threadIdx.x;
    const int blk = gtid >> 3, e = gtid & 7;
    const bool valid = blk < M * nblk;
    const int m = valid ? blk / nblk : 0, j = valid ? blk - m * nblk : 0;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v = *reinterpret_cast<const float4*>(A + (size_t)m * K + 32 * j + 4 * e);
    float s;
    int sum;
    uint32_t p0, p1;
    quant8<HP>(v, s, sum, p0, p1);
    if (valid) {
        uint8_t* rec = Aq + ((size_t)m * nblk + j) * 64;
        *reinterpret_cast<uint32_t*>(rec + 4 * e) = p0;
        *reinterpret_cast<uint32_t*>(rec + 32 + 4 * e) = p1;
        if (e == 0) {
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

// ------------------------------------------------------------------ decode GEMV (M <= 8)
//
// One workgroup of 16 waves per CU owns a contiguous range of 16-column
// tiles for up to 4 activation rows (M 5..8: one workgroup per row group of
// 4, the pair placed on the same XCD so the second read of every weight
// chunk hits its L2).  Waves 0..14 produce: a tile's K range is cut into
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
// The quantizing prologue (8 lanes per 32-block) runs on the first eight
// waves when two passes of 64 blocks cover the activations: the last waves
// of a workgroup start up to ~0.3 us after the first, and the prologue
// barrier waits for the slowest quantizer.  More blocks take all sixteen
// waves (at most kQuantPasses passes of 128).
constexpr int kQuantEarlyBlocks = 128, kQuantPasses = 4;

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
};

// One weight chunk of a wave plus its per-column metadata.  EXTRA handles
// (explicit zero points, legacy corr, scale groups smaller than a chunk)
// carry materialized per-block arrays so every load is unconditional.
template <int JG, bool EXTRA>
struct Unit {
    uint4 w;
    float sc[EXTRA ? JG : 1];
    int dl[EXTRA ? JG : 1];
    uint32_t zp;  // INT4 zero points, one byte per block
    int c;        // chunk to compute; nbg or more: none (past the end)
};

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

// The leading scalar arguments are what the first activation and weight
// loads need.  They are preloaded into SGPRs at wave launch (kernarg
// preload, 14 SGPRs), so those loads do not wait for a kernarg fetch; the
// rest of the arguments come from the struct as the code reaches them.
// Tiles per workgroup group: the first rem_t groups own base_t + 1 tiles, the
// rest base_t (ntiles = base_t * NG + rem_t).  misc = sc_shift | RG << 8 |
// pair_xcd << 10 | phases per tile << 16.  PAIR: gate and up projections
// in one launch; each output tile is the gate tile then the up tile of the
// same columns, and C = silu(gate) * up.
template <int BITS, bool HP, bool FUSED, bool EXTRA, int R, bool PAIR, bool P64>
__global__ __launch_bounds__(kDecWaves * 64) void dec_kernel(const void* act, const uint4* pW, const float* pS,
                                                             int pbase_t, int pnblk, int pM, int pnbg, int prem_t,
                                                             int pNG, int pngrp, int misc, GemvArgs args) {
    GemvArgs a = args;
    if (FUSED) a.A = static_cast<const float*>(act);
    else a.Aq = static_cast<const uint8_t*>(act);
    a.W = pW;
    a.S = pS;
    a.K = 32 * pnblk;
    a.nblk = pnblk;
    a.M = pM;
    a.nbg = pnbg;
    a.NG = pNG;
    a.ngrp = pngrp;
    a.nblk4 = (pnblk + 3) / 4 * 4;
    a.sc_shift = misc & 31;
    a.RG = (misc >> 8) & 3;
    a.pair_xcd = (misc >> 10) & 1;
    constexpr int JG = BITS == 8 ? 2 : 4;
    constexpr int PP = dec_pitch(JG);
    typedef float fvec __attribute__((ext_vector_type(JG)));
    typedef int ivec __attribute__((ext_vector_type(JG)));
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    int g, rg;
    if (a.RG == 1) {
        g = blockIdx.x;
        rg = 0;
    } else if (a.pair_xcd) {
        const int b = blockIdx.x;
        g = (b >> 4) * 8 + (b & 7);
        rg = (b >> 3) & 1;
    } else {
        g = blockIdx.x >> 1;
        rg = blockIdx.x & 1;
    }
    const int m0 = rg * 4;
    const int Mr = min(4, a.M - m0);

    // Activation loads, ahead of all other set-up in program order: at kernel
    // start the prologue's instructions are fetched cold, and timestamps put
    // the load ~1.4 us after wave start when it sat behind the set-up code.
    // K is a multiple of 32, so the rows m0.. of A are nb_rows contiguous
    // 32-float blocks, and the staged scale and sum rows (pitch nblk4) are
    // contiguous too: a block index is an offset, with no row/column split.
    const int nb_rows = Mr * a.nblk;
    uint4 av[kQuantPasses];
    uint4 r0, r1, r2, r3, r4, r5, rsa, rsq;  // named: an indexed array would live in scratch
    if (FUSED) {
        if (nb_rows > kQuantEarlyBlocks || wave < 8) {
            const float* arow = a.A + (size_t)m0 * a.K + 4 * (tid & 7);
            const bool all = nb_rows > kQuantEarlyBlocks;
            const int qb = all ? 128 : 64;  // blocks per pass
            const int npass_ld = all ? (nb_rows + 127) >> 7 : (nb_rows + 63) >> 6;
#pragma unroll
            for (int p = 0; p < kQuantPasses; ++p) {
                if (p >= npass_ld) break;
                const int blk = min(p * qb + (tid >> 3), nb_rows - 1);
                av[p] = *reinterpret_cast<const uint4*>(arow + 32 * blk);
            }
        }
    } else {
        // Records of rows m0.. are contiguous: nb_rows*4 uint4, then the
        // scale and sum(q) rows as uint4 (Mr * nblk4 / 4 each).
        const uint4* rsrc = reinterpret_cast<const uint4*>(a.Aq + (size_t)m0 * a.nblk * 64);
        const int nrec = nb_rows * 4, nmeta = Mr * a.nblk4 / 4;
        // With one or two rows (block pairs) only the groups of 1024
        // records that hold work are loaded; with more rows every group is
        // (branches there cost more than the clamped loads).
        r0 = rsrc[min(tid, nrec - 1)];
        r1 = rsrc[min(1024 + tid, nrec - 1)];
        r2 = rsrc[min(2048 + tid, nrec - 1)];
        if (!P64 || nrec > 3072) {
            r3 = rsrc[min(3072 + tid, nrec - 1)];
            r4 = rsrc[min(4096 + tid, nrec - 1)];
            r5 = rsrc[min(5120 + tid, nrec - 1)];
        }
        const int mi = min(tid, nmeta - 1);
        rsa = *reinterpret_cast<const uint4*>(a.Sa + (size_t)m0 * a.nblk4 + 4 * mi);
        rsq = *reinterpret_cast<const uint4*>(a.Sq + (size_t)m0 * a.nblk4 + 4 * mi);
    }
    __builtin_amdgcn_sched_barrier(0);

    const int base_t = pbase_t, rem_t = prem_t;
    const int t_begin = g * base_t + min(g, rem_t);
    const int nT = base_t + (g < rem_t ? 1 : 0);
    const int nbg = a.nbg;
    const int npw = misc >> 16;                // phases per tile: ceil(nbg / 15)
    const int U = nT * npw * (PAIR ? 2 : 1);  // phases of this workgroup

    const DecLds lay = dec_lds(min(a.M, 4), a.nblk, JG, P64);
    uint8_t* recs = smem + lay.recs;
    float* sa_l = reinterpret_cast<float*>(smem + lay.sa);
    int* sq_l = reinterpret_cast<int*>(smem + lay.sq);
    float* fbuf = reinterpret_cast<float*>(smem + lay.fbuf);  // [2][64][PP]

    const int col = lane & 15, grp = lane >> 4;
    const int me = min(grp, Mr - 1);

    // Load cursor, kept incrementally: one scalar unit serves the CU's
    // sixteen waves, which reach their scalar work together after each
    // barrier, so every scalar instruction per unit lengthens every phase.
    // The next unit is chunk ld_c (clamped to the tile's last chunk) of local
    // tile ld_t, ld_rem units before the tile ends; ld_w, ld_s and ld_m index
    // the tile's weights, scales and per-block metadata.  Past the end ld_c
    // is out of range (no work) and the loads re-read the last tile.
    //
    // A producer with no chunk in a tile's short last phase still fills its
    // ring slot.  That load's data is never used, so its weight address is
    // the chunk this producer loads next in the following tile (chunk
    // wave + 15, requested two phases later): the slot warms L2 for it.  The
    // tiles of a workgroup are contiguous, so that is chunk nbg + wave + 15
    // from the current tile.  On the last tile (and for gate/up pairs, whose
    // next tile lies in the other array) the load re-reads the tile's last
    // chunk instead, so every address stays inside the workgroup's tiles.
    int ld_c = wave, ld_rem = npw, ld_t = 0, ld_sel = 0;  // ld_sel: up tile of a pair
    uint32_t ld_w = (uint32_t)t_begin * nbg * 64;
    uint32_t ld_s = (uint32_t)t_begin * a.ngrp * 16;
    uint32_t ld_m = (uint32_t)t_begin * nbg * 16;
    const int pf_c = nbg + kProducers + wave;
    const bool pf = !PAIR && npw >= 2 && wave + kProducers < nbg;
    int ld_idle = (pf && nT > 1) ? pf_c : nbg - 1;  // weight chunk of a load with no work
    auto load_unit = [&](Unit<JG, EXTRA>& p) {
        const int c = min(ld_c, nbg - 1);
        const int cw = ld_c < nbg ? ld_c : ld_idle;
        uint32_t wi = ld_w + cw * 64 + lane;                               // weight uint4 index
        uint32_t mi = ld_m + c * 16 + col;                                 // per-block metadata (EXTRA)
        uint32_t si = ld_s + (uint32_t)((c * JG) >> a.sc_shift) * 16 + col;  // scale index
        // Opaque to the optimizer, so the loads are not split into
        // uniform-address copies on branches of their own.
        asm("" : "+v"(wi), "+v"(mi), "+v"(si));
        const bool up = PAIR && ld_sel;
        p.w = (up ? a.W2 : a.W)[wi];
        if (EXTRA) {
            const fvec sv = *reinterpret_cast<const fvec*>((up ? a.S2 : a.S) + (size_t)mi * JG);
            const ivec dv = *reinterpret_cast<const ivec*>((up ? a.D2 : a.D) + (size_t)mi * JG);
#pragma unroll
            for (int jb = 0; jb < JG; ++jb) {
                p.sc[EXTRA ? jb : 0] = sv[jb];
                p.dl[EXTRA ? jb : 0] = dv[jb];
            }
            if (JG == 4) p.zp = *reinterpret_cast<const uint32_t*>((up ? a.Z2 : a.Z) + (size_t)mi * 4);
        } else {
            p.sc[0] = (up ? a.S2 : a.S)[si];
        }
        p.c = ld_c;
        ld_c += kProducers;
        if (--ld_rem == 0) {
            ld_rem = npw;
            if (PAIR && ld_sel == 0 && ld_t < nT) {
                ld_sel = 1;  // the same tile's up projection
                ld_c = wave;
            } else {
                if (PAIR) ld_sel = 0;
                if (++ld_t < nT) {
                    ld_c = wave;
                    ld_w += nbg * 64;
                    ld_s += a.ngrp * 16;
                    ld_m += nbg * 16;
                    if (ld_t + 1 == nT) ld_idle = nbg - 1;
                } else {
                    ld_c = 1 << 24;
                }
            }
        }
    };

    // ---------------- prologue
    // The activation loads went out first (above); the first R weight units
    // follow, then the activations are quantized (or their records copied)
    // into LDS while the weights stream in.  The scheduling barriers keep
    // this issue order.
    auto store_acts = [&]() {
        if (FUSED) {
            const bool all = nb_rows > kQuantEarlyBlocks;
            const int qb = all ? 128 : 64;  // blocks per pass
            const int npass = all ? (nb_rows + 127) >> 7 : wave < 8 ? (nb_rows + 63) >> 6 : 0;
#pragma unroll
            for (int p = 0; p < kQuantPasses; ++p) {
                if (p >= npass) break;
                const int blk = p * qb + (tid >> 3), e = tid & 7;
                float s;
                int sum;
                uint32_t p0, p1;
                quant8<HP>(make_float4(__uint_as_float(av[p].x), __uint_as_float(av[p].y),
                                       __uint_as_float(av[p].z), __uint_as_float(av[p].w)),
                           s, sum, p0, p1);
                if (blk < nb_rows) {
                    const int m = (blk >= a.nblk) + (blk >= 2 * a.nblk) + (blk >= 3 * a.nblk), j = blk - m * a.nblk;
                    if (P64) {
                        // Lane e holds bytes 4(e&1).. of k-octet e>>1: the
                        // slot's zero half, then the octet.
                        uint32_t* sh = reinterpret_cast<uint32_t*>(recs + m * lay.rec_pitch + j * 128 +
                                                                   (e >> 1) * 16) + (e & 1);
                        sh[0] = 0u;
                        sh[2] = p0;
                        sh[16] = 0u;  // l octets, 64 B further
                        sh[18] = p1;
                    } else {
                        // [chunk][h, l][k-octet][block of the chunk] of 8
                        // bytes: a lane's A operands for a chunk are 8 JG
                        // contiguous bytes.
                        uint8_t* rec = recs + m * lay.rec_pitch + (j / JG) * (JG * 64) + (e >> 1) * (JG * 8) +
                                       (j % JG) * 8 + 4 * (e & 1);
                        *reinterpret_cast<uint32_t*>(rec) = p0;
                        *reinterpret_cast<uint32_t*>(rec + JG * 32) = p1;
                    }
                    if (e == 0) {
                        sa_l[m * lay.sa_pitch + j] = s;
                        sq_l[m * lay.sa_pitch + j] = (EXTRA ? -1 : -8) * sum;
                    }
                }
            }
        } else {
            // Rows land at the padded LDS pitches.
            const int nrec = nb_rows * 4, nmeta = Mr * a.nblk4 / 4;
            const int L = a.nblk * 4;
            auto put = [&](int i, const uint4& v) {
                i = min(i, nrec - 1);
                const int m = (i >= L) + (i >= 2 * L) + (i >= 3 * L);
                if (P64) {
                    // Source uint4 q of a block: h or l (q >> 1) octets
                    // 2(q & 1) and 2(q & 1) + 1, each into its slot.
                    const int r = i - m * L, j = r >> 2, q = r & 3;
                    uint4* slot = reinterpret_cast<uint4*>(recs + m * lay.rec_pitch + j * 128 + (q >> 1) * 64 +
                                                           (q & 1) * 32);
                    slot[0] = make_uint4(0u, 0u, v.x, v.y);
                    slot[1] = make_uint4(0u, 0u, v.z, v.w);
                } else {
                    // Source uint4 q of a block: h or l (q >> 1) octets
                    // 2(q & 1) and 2(q & 1) + 1, each to its place in the
                    // [chunk][h, l][k-octet][block] layout.
                    const int r = i - m * L, j = r >> 2, q = r & 3;
                    uint8_t* o = recs + m * lay.rec_pitch + (j / JG) * (JG * 64) + (q >> 1) * (JG * 32) +
                                 2 * (q & 1) * (JG * 8) + (j % JG) * 8;
                    *reinterpret_cast<uint2*>(o) = make_uint2(v.x, v.y);
                    *reinterpret_cast<uint2*>(o + JG * 8) = make_uint2(v.z, v.w);
                }
            };
            // Threads past the end rewrite the last element with the value
            // they loaded from it; with block pairs, groups of 1024 records
            // without work are skipped (up to 3072 such stores to one LDS
            // address otherwise).
            put(tid, r0);
            put(1024 + tid, r1);
            put(2048 + tid, r2);
            if (!P64 || nrec > 3072) {
                put(3072 + tid, r3);
                put(4096 + tid, r4);
                put(5120 + tid, r5);
            }
            const int mi = min(tid, nmeta - 1);
            const int mm = (4 * mi >= a.nblk4) + (4 * mi >= 2 * a.nblk4) + (4 * mi >= 3 * a.nblk4);
            const int md = mi + mm * ((lay.sa_pitch - a.nblk4) >> 2);
            reinterpret_cast<uint4*>(sa_l)[md] = rsa;
            const uint32_t f = EXTRA ? 0xFFFFFFFFu : 0xFFFFFFF8u;  // -1 or -8
            reinterpret_cast<uint4*>(sq_l)[md] = make_uint4(f * rsq.x, f * rsq.y, f * rsq.z, f * rsq.w);
        }
        {
            uint32_t* cst = reinterpret_cast<uint32_t*>(smem + lay.consts);
            if (P64) {
                // [8 zeros][8 bytes of 64], then zeros; and each record row's
                // closing zero slot.
                if (tid < 128) cst[tid] = (tid == 2 || tid == 3) ? 0x40404040u : 0u;
                if (tid < 4 * Mr) {
                    uint32_t* z = reinterpret_cast<uint32_t*>(recs + (tid >> 2) * lay.rec_pitch + a.nblk * 128);
                    z[tid & 3] = 0u;
                }
            } else if (tid < 128) {
                cst[tid] = tid < 64 ? 0x40404040u : 0u;  // [0,256) bytes of 64, [256,512) zeros
            }
        }
    };

    if (wave == kChainWave) {
        // ================= chain wave
        // Its fold is one dependent FMA chain per output and paces the
        // phases: first pick of the SIMD's issue slots over the producers.
        __builtin_amdgcn_s_setprio(3);
        store_acts();
        lds_barrier();
        // Lane (row me, column col) of the current tile.
        const float* sa_row = sa_l + me * lay.sa_pitch;
        const bool tail_pad = a.nblk != nbg * JG;  // the last chunk has padding blocks
        float acc = 0.0f, gate = 0.0f;
        unsigned long long best = 0;
        int pr_t = 0, pr_p = 0, pr_sel = 0;
        for (int u = 0; u < U; ++u) {
            lds_barrier();
            const float* fp = fbuf + ((u & 1) * 64 + lane) * PP;
            const int c0 = kProducers * pr_p;
            const float* sp = sa_row + c0 * JG;
            if (c0 + kProducers < nbg || (c0 + kProducers == nbg && !tail_pad)) {
                // Full phase: every block is real.  All fifteen chunks'
                // reads, then the FMAs: right after the barrier the reads
                // queue behind the producers' operand reads (~0.3 us), so
                // one wait instead of one per group of chunks.
                fvec fv[kProducers], sv[kProducers];
#pragma unroll
                for (int i = 0; i < kProducers; ++i) {
                    fv[i] = *reinterpret_cast<const fvec*>(fp + i * JG);
                    sv[i] = *reinterpret_cast<const fvec*>(sp + i * JG);
                }
#pragma unroll
                for (int i = 0; i < kProducers; ++i) {
#pragma unroll
                    for (int jb = 0; jb < JG; ++jb) acc = __builtin_fmaf(sv[i][jb], fv[i][jb], acc);
                }
            } else {
                // The tile's last phase: whole chunks two at a time with
                // wide reads, then the blocks of a padded last chunk.
                const int nb = a.nblk - c0 * JG, nwc = nb / JG;
                int i = 0;
                for (; i + 2 <= nwc; i += 2) {
                    const fvec f0 = *reinterpret_cast<const fvec*>(fp + i * JG);
                    const fvec s0 = *reinterpret_cast<const fvec*>(sp + i * JG);
                    const fvec f1 = *reinterpret_cast<const fvec*>(fp + (i + 1) * JG);
                    const fvec s1 = *reinterpret_cast<const fvec*>(sp + (i + 1) * JG);
#pragma unroll
                    for (int jb = 0; jb < JG; ++jb) acc = __builtin_fmaf(s0[jb], f0[jb], acc);
#pragma unroll
                    for (int jb = 0; jb < JG; ++jb) acc = __builtin_fmaf(s1[jb], f1[jb], acc);
                }
                if (i < nwc) {
                    const fvec f0 = *reinterpret_cast<const fvec*>(fp + i * JG);
                    const fvec s0 = *reinterpret_cast<const fvec*>(sp + i * JG);
#pragma unroll
                    for (int jb = 0; jb < JG; ++jb) acc = __builtin_fmaf(s0[jb], f0[jb], acc);
                    ++i;
                }
                for (int b = i * JG; b < nb; ++b) acc = __builtin_fmaf(sp[b], fp[b], acc);
            }
            if (++pr_p == npw) {
                if (PAIR && pr_sel == 0) {
                    gate = acc;  // the up tile of the same columns follows
                    pr_sel = 1;
                } else {
                    // silu(g) = g / (1 + exp(-g)) (qwen35_decoder.cpp:129),
                    // times the up projection (qwen35_decoder.cpp:408).
                    const float v = PAIR ? gate / (1.0f + expf(-gate)) * acc : acc;
                    if (grp < Mr) {
                        const int n = (t_begin + pr_t) * 16 + col;
                        a.C[(size_t)(m0 + grp) * a.N + n] = v;
                        if (!PAIR && a.idx) {
                            const unsigned long long k = argmax_key(acc, n);
                            best = k > best ? k : best;
                        }
                    }
                    if (PAIR) pr_sel = 0;
                    ++pr_t;
                }
                acc = 0.0f;
                pr_p = 0;
            }
        }
        if (!PAIR && a.idx) {
            // Row maximum over the lanes of each row (lanes 16r..16r+15).
#pragma unroll
            for (int s = 1; s < 16; s <<= 1) {
                const unsigned long long o = __shfl_xor(best, s, 16);
                best = o > best ? o : best;
            }
            {
                // Argmax without a second launch: each workgroup merges its
                // row keys into idx_key with device-scope atomic max, waits
                // for them, then takes a ticket; the workgroup holding the
                // last ticket swaps the merged keys back to zero (re-arming
                // them for the next call) and writes the indices.
                if (col == 0 && grp < Mr) (void)atomicMax(a.key + m0 + grp, best);
                __builtin_amdgcn_s_waitcnt(0);
                unsigned int t = 0;
                if (lane == 0) t = atomicAdd(a.ticket, 1u);
                t = __shfl(t, 0);
                if (t == gridDim.x - 1 && lane < a.M) {
                    const unsigned long long k = atomicExch(a.key + lane, 0ull);
                    a.idx[lane] = (int64_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
                    if (lane == 0) atomicExch(a.ticket, 0u);
                }
            }
        }
        return;
    }

    // ================= producers (waves 0..14)
    // Quantizing in the prologue: the first weight units stream in while it
    // runs.  Copying staged records (up to 96 KB per workgroup): the copy
    // goes first, since weight requests issued beside it slowed it down
    // (three and four rows: 11.8 -> 11.3 us).
    Unit<JG, EXTRA> ring[R];
    if (!FUSED) {
        store_acts();
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int d = 0; d < R; ++d) load_unit(ring[d]);
    __builtin_amdgcn_sched_barrier(0);
    if (FUSED) store_acts();
    lds_barrier();

    // A operand: lane row arow = 4 * group + slot, k-octet kq.  Slots 0 and
    // 1 are the h and l bytes; slots 2 and 3 are rows of 64, so their two
    // results add up to the 128 * sum(b) term.  Output lane (col, grp) holds
    // row grp.  The LDS sums of q hold the zero-point term's factor: -sum(q)
    // for explicit zero points, -8 * sum(q) for the default zero point 8.
    const int arow = lane & 15, arg = arow >> 2, ars = arow & 3, kq = lane >> 4;
    const bool is_data = ars < 2 && arg < Mr;
    const int data_base = lay.recs + arg * lay.rec_pitch + ars * (JG * 32) + kq * (JG * 8);
    const int const_base = lay.consts + ((ars >= 2 && arg < Mr) ? 0 : 256) + kq * (JG * 8);
    // P64: A row r = 8 * activation row + 4 * (block of the pair) + slot,
    // read as 16 bytes from the zero-padded octet slots ([octet | zeros] for
    // the pair's first block, [zeros | octet] for its second).  Output lane
    // (col, grp): activation row grp >> 1, block 2 * mi + (grp & 1).
    const int p_row = arow >> 3, p_sel = (arow >> 2) & 1;
    const bool p_data = ars < 2 && p_row < Mr;
    const int p_data_base = lay.recs + p_row * lay.rec_pitch + ars * 64 + kq * 16 + p_sel * 128 + 8 - 8 * p_sel;
    const int p_const_base = lay.consts + ((ars >= 2 && p_row < Mr) ? 8 - 8 * p_sel : 16);
    const int o_row = min(grp >> 1, Mr - 1), o_sel = grp & 1;
    float* const p_fout = fbuf + (col + 16 * (grp >> 1)) * PP + wave * JG + o_sel;

    for (int u0 = 0; u0 < U; u0 += R) {
#pragma unroll
        for (int d = 0; d < R; ++d) {
            const bool live = u0 + d < U;  // uniform over the workgroup
            const int c = ring[d].c;
            const int buf = (u0 + d) & 1;
            if (P64 && c < nbg) {
                const Unit<JG, EXTRA>& cur = ring[d];
                const int abase = p_data ? p_data_base + c * JG * 128 : p_const_base;
                int2 nsq2 = make_int2(0, 0);  // this lane's block in each pair
                if (BITS == 4) {
                    const int* q = sq_l + o_row * lay.sa_pitch + c * 4 + o_sel;
                    nsq2 = make_int2(q[0], q[2]);
                }
                float fo[JG / 2];
#pragma unroll
                for (int mi = 0; mi < JG / 2; ++mi) {
                    // Blocks past nblk (last chunk) read padding; the chain
                    // never folds them.
                    uint4 bop = cur.w;
                    if (BITS == 4) {
                        const uint64_t b0 = unpack_b(cur.w, 2 * mi, 4), b1 = unpack_b(cur.w, 2 * mi + 1, 4);
                        bop = make_uint4((uint32_t)b0, (uint32_t)(b0 >> 32), (uint32_t)b1, (uint32_t)(b1 >> 32));
                    }
                    const uint8_t* ap = smem + abase + (p_data ? mi * 256 : 0);
                    const uint2 alo = *reinterpret_cast<const uint2*>(ap);
                    const uint2 ahi = *reinterpret_cast<const uint2*>(ap + 8);
                    const v4i dd = mfma64(make_uint4(alo.x, alo.y, ahi.x, ahi.y), bop);
                    int cs = HP ? (dd[0] * 256 + dd[1]) + (dd[2] + dd[3]) : dd[0];
                    if (BITS == 4) {
                        const int nsq = mi == 0 ? nsq2.x : nsq2.y;
                        cs += EXTRA ? (int)(int8_t)((o_sel ? cur.zp >> 8 : cur.zp) >> (16 * mi)) * nsq : nsq;
                    }
                    float sc = cur.sc[0];
                    if (EXTRA) {
                        // Values first, then the lane's pick: a select
                        // between array elements would index the unit in
                        // memory.
                        const int dl0 = cur.dl[EXTRA ? 2 * mi : 0], dl1 = cur.dl[EXTRA ? 2 * mi + 1 : 0];
                        const float sc0 = cur.sc[EXTRA ? 2 * mi : 0], sc1 = cur.sc[EXTRA ? 2 * mi + 1 : 0];
                        cs += (HP ? 256 : 1) * (o_sel ? dl1 : dl0);
                        sc = o_sel ? sc1 : sc0;
                    }
                    fo[mi] = (float)cs * sc;
                }
                // Both results in one LDS instruction (ds_write2_b32): the
                // phase is bounded by LDS instruction issue, ~8 CU cycles each.
#pragma unroll
                for (int mi = 0; mi < JG / 2; ++mi) p_fout[buf * 64 * PP + 2 * mi] = fo[mi];
            } else if (!P64 && c < nbg) {
                const Unit<JG, EXTRA>& cur = ring[d];
                const int abase = is_data ? data_base + c * JG * 64 : const_base;
                // The chunk's JG A operands of this lane: 8 JG contiguous bytes.
                uint4 av4[JG / 2];
#pragma unroll
                for (int h = 0; h < JG / 2; ++h) av4[h] = *reinterpret_cast<const uint4*>(smem + abase + 16 * h);
                int4 sqv = make_int4(0, 0, 0, 0);
                if (BITS == 4) sqv = *reinterpret_cast<const int4*>(sq_l + me * lay.sa_pitch + c * 4);
                fvec fo;
#pragma unroll
                for (int jb = 0; jb < JG; ++jb) {
                    // Blocks past nblk (last chunk) read padding; the chain
                    // never folds them.
                    const uint64_t bop = unpack_b(cur.w, jb, BITS);
                    const uint4& a2 = av4[jb >> 1];
                    const uint64_t aop = (jb & 1) ? ((uint64_t)a2.w << 32 | a2.z) : ((uint64_t)a2.y << 32 | a2.x);
                    const v4i dd = mfma16(aop, bop);
                    int cs = HP ? (dd[0] * 256 + dd[1]) + (dd[2] + dd[3]) : dd[0];
                    if (BITS == 4) {
                        const int nsq = jb == 0 ? sqv.x : jb == 1 ? sqv.y : jb == 2 ? sqv.z : sqv.w;
                        cs += EXTRA ? (int)(int8_t)(cur.zp >> (8 * jb)) * nsq : nsq;
                    }
                    if (EXTRA) cs += (HP ? 256 : 1) * cur.dl[EXTRA ? jb : 0];
                    fo[jb] = (float)cs * cur.sc[EXTRA ? jb : 0];
                }
                *reinterpret_cast<fvec*>(fbuf + (buf * 64 + lane) * PP + wave * JG) = fo;
            }
            load_unit(ring[d]);
            __builtin_amdgcn_sched_barrier(0);
            if (live) lds_barrier();
        }
    }
}

// ------------------------------------------------------------------ generic rows kernel (M > 8)
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

// ------------------------------------------------------------------ prefill GEMM (M > 8)
//
// One workgroup of 8 waves computes 128 rows x 16*CT columns over all of K.
// Wave w owns rows 32 (w & 3) .. +31 and column half w >> 2 (the first
// (CT+1)/2 tiles or the other CT/2), so each SIMD holds one wave of each
// half.  Per 32-block, H = sum(h*b) comes from one MFMA, (H << 8) + 128*S is
// the accumulator input of the l-byte MFMA, which then holds the exact block
// integer cs, and the lane folds acc = fma(s_a, f32(cs) * s_b, acc) in block
// order.  Pairs of tiles run on v_mfma_i32_32x32x32_i8, an odd last tile on
// v_mfma_i32_16x16x32_i8.
//
// Operands reach LDS by direct global->LDS loads (global_load_lds_dwordx4,
// 16 bytes per lane to LDS address M0 + 16*lane) through a ring of
// kPfStages stages.  A stage holds one chunk (two blocks): the CT weight
// tiles (1 KB each; the decode layout is the MFMA B operand), their weight
// sums and scales (the shared part, loaded by all waves together), and each
// wave's activation record.  The compiler does not see these loads: every
// wave waits for its own with an explicit vmcnt, then the workgroup barrier
// publishes the stage.
//
// INT4 weights (BITS 4) take the same core.  A stage is one INT4 chunk (four
// blocks, 1 KB per tile), loaded raw into chunk 0's weight area; its scales
// and zero points go to one raw area shared by both stages.  After the
// stage barrier all 512 threads expand it in place: per byte, b = nibble -
// zp as a signed byte ((n | 0x80) - zp) ^ 0x80, chunk 0 getting blocks 0-1
// and chunk 1 blocks 2-3 in the INT8 chunk layout, plus 128 * sum(b) per
// (column, block) for the two-pass product and the scales in the INT8
// chunk layout.  A second barrier publishes the expanded stage.

constexpr int kPfWaves = 8, kPfRows = 16 * kPfWaves;
// Ring of kPfStages stages of kPfChunks chunks each.
constexpr int kPfStages = 2, kPfChunks = 2;
// Activation record per (16-row tile, chunk): [block 2][lane 64][h 8 B, l 8 B]
// in MFMA A-operand order (lane: row lane&15, k-octet lane>>4), then the
// block scales [block 2][row 16] float.
constexpr int kRecA = 2048, kRecBytes = kRecA + 128;

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
// per tile][block or group scales][8 activation records].  INT4 adds the raw
// area after the two stages: group scales (SCM 1, 64 B per tile) or block
// scales then zero points (SCM 2, 256 + 64 B per tile), in whole KB.
template <int CT, int SCM, int BITS>
struct PfLayout {
    static constexpr int kWS = CT * 1024;
    static constexpr int kSB = kWS + CT * 128;
    static constexpr int kShared = kSB + (SCM == 2 ? CT * 128 : SCM == 1 ? CT * 64 : 0);
    static constexpr int kA = kShared;
    static constexpr int kChunk = kA + kPfWaves * kRecBytes;
    static constexpr int kStage = kPfChunks * kChunk;
    static constexpr int kRawZ = CT * 256;  // SCM 2: zero points after the block scales
    static constexpr int kRawUsed = BITS == 8 ? 0 : SCM == 2 ? CT * 320 : SCM == 1 ? CT * 64 : 0;
    static constexpr int kRaw = (kRawUsed + 1023) / 1024 * 1024;
    static constexpr int kRawOff = kPfStages * kStage;
    // DMA units of 1 KB per stage (INT8: per chunk): INT8 the chunk's shared
    // part, INT4 the CT raw tiles and the raw area.
    static constexpr int kUnits = BITS == 8 ? (kShared + 1023) / 1024 : CT + kRaw / 1024;
    static constexpr int kPerWave = (kUnits + kPfWaves - 1) / kPfWaves;
    static constexpr int kBytes = kRawOff + kRaw;
    static_assert(kShared % 64 == 0 && kBytes <= 160 * 1024, "layout");
};

__device__ inline uint32_t lds_address(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 16 bytes per lane from global `src` to LDS byte address lds + 16*lane.
__device__ inline void dma16(const void* src, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

// s_waitcnt immediate: vmcnt(n), no wait on the other counters.
__host__ __device__ constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00; }

template <int BITS, bool HP, int SCM, int CT>
__global__ __launch_bounds__(kPfWaves * 64) void prefill_kernel(PfArgs a) {
    using L = PfLayout<CT, SCM, BITS>;
    extern __shared__ __align__(16) char pf_lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int col = lane & 15, grp = lane >> 4;
    // Wave w: row pair w&3 (two 16-row tiles) and column half w>>2, so each
    // SIMD (waves w and w+4) holds one wave of each half.
    const int rp = wave & 3, half = wave >> 2;
    const int t0 = blockIdx.x * CT;
    const int rt0 = blockIdx.y * kPfWaves + 2 * rp;
    const bool active = rt0 * 16 < a.M;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(pf_lds));
    const int nch = a.nch;
    const int nst = (nch + kPfChunks - 1) / kPfChunks;
    const bool odd = a.nblk & 1;

    // Shared part of a chunk (INT8) or stage (INT4): slot k of this wave
    // loads the 1 KB at x0, u = k * kPfWaves + wave (clamped), lane bytes
    // x0 + 16*lane.  INT8: x0 = min(u * 1024, kShared - 1024) in the chunk
    // (overlapping slots write equal bytes).  INT4: raw tile u of the stage
    // into chunk 0's weight area, or KB u - CT of the raw area.
    const char* src0[L::kPerWave];
    uint32_t step[L::kPerWave], gstep[L::kPerWave], x0s[L::kPerWave];
    bool to_raw[L::kPerWave];
#pragma unroll
    for (int k = 0; k < L::kPerWave; ++k) {
        const int u = min(k * kPfWaves + wave, L::kUnits - 1);
        const int x0 = min(u * 1024, L::kShared - 1024);
        const int x = x0 + 16 * lane;
        x0s[k] = (uint32_t)x0;
        gstep[k] = 0;
        to_raw[k] = false;
        if (BITS == 4) {
            if (u < CT) {
                const int tc = min(t0 + u, a.ntiles - 1);
                src0[k] = a.W + (size_t)tc * a.nbg * 1024 + 16 * lane;
                step[k] = 1024;
                x0s[k] = (uint32_t)(u * 1024);
            } else {
                const int y = (u - CT) * 1024 + 16 * lane;
                to_raw[k] = true;
                x0s[k] = (uint32_t)(L::kRawOff + (u - CT) * 1024);
                src0[k] = a.S;  // padding lanes: any valid source
                step[k] = 0;
                if (SCM == 2 && y < L::kRawZ) {
                    const int tc = min(t0 + (y >> 8), a.ntiles - 1);
                    src0[k] = a.S + (size_t)tc * a.nbg * 256 + (y & 255);
                    step[k] = 256;
                } else if (SCM == 2 && y < L::kRawUsed) {
                    const int yz = y - L::kRawZ;
                    const int tc = min(t0 + (yz >> 6), a.ntiles - 1);
                    src0[k] = a.Z + (size_t)tc * a.nbg * 64 + (yz & 63);
                    step[k] = 64;
                } else if (SCM == 1 && y < L::kRawUsed) {
                    const int tc = min(t0 + (y >> 6), a.ntiles - 1);
                    src0[k] = a.S + (size_t)tc * a.ngrp * 64 + (y & 63);
                    gstep[k] = 64;
                }
            }
        } else if (x < L::kWS) {
            const int tc = min(t0 + (x >> 10), a.ntiles - 1);
            src0[k] = a.W + (size_t)tc * nch * 1024 + (x & 1023);
            step[k] = 1024;
        } else if (x < L::kSB) {
            const int y = x - L::kWS;
            const int tc = min(t0 + (y >> 7), a.ntiles - 1);
            src0[k] = a.WS + (size_t)tc * nch * 128 + (y & 127);
            step[k] = 128;
        } else if (SCM == 2) {
            const int y = x - L::kSB;
            const int tc = min(t0 + (y >> 7), a.ntiles - 1);
            src0[k] = a.S + (size_t)tc * nch * 128 + (y & 127);
            step[k] = 128;
        } else {
            const int y = x - L::kSB;
            const int tc = min(t0 + (y >> 6), a.ntiles - 1);
            src0[k] = a.S + (size_t)tc * a.ngrp * 64 + (y & 63);
            step[k] = 0;
            gstep[k] = 64;
        }
    }
    // This wave's two activation records per chunk.
    const char* rec0 = a.R + (size_t)rt0 * nch * kRecBytes + 16 * lane;
    const size_t rec_step = (size_t)nch * kRecBytes;  // next row tile

    // Load d of this wave's kDmaChunk loads of chunk c into the chunk region
    // at LDS address cbase: the shared slots, then 3 per activation record.
    constexpr int kDmaChunk = L::kPerWave + 6;
    // INT4: only chunk 0 of a stage (first) carries the stage's shared loads.
    auto dma_slot = [&](int c, uint32_t cbase, int d, bool first) {
        if (d < L::kPerWave) {
            if (BITS == 8) {
                const size_t g = SCM == 1 ? (size_t)((2 * c) >> a.sc_shift) : 0;
                dma16(src0[d] + (size_t)c * step[d] + g * gstep[d], cbase + x0s[d]);
            } else if (first) {
                const int sg = c >> 1;
                const size_t g = SCM == 1 ? (size_t)((4 * sg) >> a.sc_shift) : 0;
                dma16(src0[d] + (size_t)sg * step[d] + g * gstep[d], (to_raw[d] ? lds0 : cbase) + x0s[d]);
            }
        } else {
            const int e = d - L::kPerWave, r = e / 3, part = e % 3;
            const int off = part == 0 ? 0 : part == 1 ? 1024 : 1152;
            dma16(rec0 + r * rec_step + (size_t)c * kRecBytes + off,
                  cbase + (uint32_t)(L::kA + (2 * rp + r) * kRecBytes + off));
        }
    };
    auto issue_chunk = [&](int c, uint32_t cbase, bool first) {
#pragma unroll
        for (int d = 0; d < kDmaChunk; ++d) dma_slot(c, cbase, d, first);
    };
    auto issue_stage = [&](int g, int buf) {
        const uint32_t sbase = lds0 + (uint32_t)(buf * L::kStage);
#pragma unroll
        for (int cc = 0; cc < kPfChunks; ++cc) {
            const int c = g * kPfChunks + cc;
            if (c < nch) issue_chunk(c, sbase + (uint32_t)(cc * L::kChunk), cc == 0);
        }
    };

    // INT4: expands stage buffer buf in place (all threads; a workgroup
    // barrier must follow).  Wave w takes tiles w, w + 8, ...; lane l holds
    // weight lane l of the tile (column l & 15, k-octet l >> 4), so the LDS
    // reads and writes are linear.  The nibble sums of a column's four
    // octets (one per 16-lane row) meet by row swaps.
    auto expand = [&](int buf) {
        if constexpr (BITS == 4) {
            char* sb = pf_lds + buf * L::kStage;
            const char* raw = pf_lds + L::kRawOff;
            const int c = lane & 15, o = lane >> 4, cc = o & 1;
            for (int t = wave; t < CT; t += kPfWaves) {
                const int wl = t * 1024 + 16 * lane;
                const uint4 w = *reinterpret_cast<const uint4*>(sb + wl);
                const uint32_t z = SCM == 2 ? *reinterpret_cast<const uint32_t*>(raw + L::kRawZ + t * 64 + 4 * c)
                                            : 0x08080808u;
                const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
                uint32_t lo[4], hi[4], nsum[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const uint32_t zr = SCM == 2 ? ((z >> (8 * b)) & 0xFFu) * 0x01010101u : 0x08080808u;
                    lo[b] = (((wv[b] & 0x0F0F0F0Fu) | 0x80808080u) - zr) ^ 0x80808080u;
                    hi[b] = ((((wv[b] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - zr) ^ 0x80808080u;
                    nsum[b] = __builtin_amdgcn_udot8(wv[b], 0x11111111u, 0u, false);  // <= 120
                }
                *reinterpret_cast<uint4*>(sb + wl) = make_uint4(lo[0], hi[0], lo[1], hi[1]);
                *reinterpret_cast<uint4*>(sb + L::kChunk + wl) = make_uint4(lo[2], hi[2], lo[3], hi[3]);
                // Per-column nibble sums of blocks (0, 1) and (2, 3), two per
                // dword, summed over the four rows (octets).
                uint32_t ps[2] = {nsum[0] | nsum[1] << 16, nsum[2] | nsum[3] << 16};
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const auto s32 = __builtin_amdgcn_permlane32_swap(ps[q], ps[q], false, false);
                    const uint32_t y = s32[0] + s32[1];
                    const auto s16 = __builtin_amdgcn_permlane16_swap(y, y, false, false);
                    ps[q] = s16[0] + s16[1];
                }
                char* cb = sb + cc * L::kChunk;
                if (o < 2) {
                    // Row o: 128 * sum(n - zp) of chunk o's two blocks.
                    const uint32_t p2 = cc ? ps[1] : ps[0];
                    const uint32_t zz = SCM == 2 ? z >> (16 * cc) : 0x0808u;
                    const int s0 = (int)(p2 & 0xFFFFu) - 32 * (int)(zz & 0xFFu);
                    const int s1 = (int)(p2 >> 16) - 32 * (int)((zz >> 8) & 0xFFu);
                    *reinterpret_cast<int2*>(cb + L::kWS + t * 128 + 8 * c) = make_int2(128 * s0, 128 * s1);
                } else if (SCM == 2) {
                    *reinterpret_cast<float2*>(cb + L::kSB + t * 128 + 8 * c) =
                        *reinterpret_cast<const float2*>(raw + t * 256 + 16 * c + 8 * cc);
                } else if (SCM == 1) {
                    *reinterpret_cast<float*>(cb + L::kSB + t * 64 + 4 * c) =
                        *reinterpret_cast<const float*>(raw + t * 64 + 4 * c);
                }
            }
        }
    };

    // The whole K loop of one column half (CTW tiles from WG tile toff) on
    // v_mfma_i32_32x32x32_i8: the wave's two 16-row records are its 32 rows
    // and pairs of its tiles are 32-column groups, one MFMA per (group,
    // 32-block) at the full INT8 rate (twice the 16x16x32 rate).  An odd
    // last tile of the half takes 16x16x32 MFMAs on the 16-row records.
    // Per (group, block) the h-byte MFMA's result, shifted left by 8 plus
    // 128 * sum(b), is the l-byte MFMA's accumulator input, so that MFMA
    // holds the exact block integer cs, and the lane folds
    // acc = fma(s_a, f32(cs) * s_b, acc) in block order.
    // Lane l: A row / output column c32 = l & 31, k half kh = l >> 5.  The
    // operands come from the same LDS layout: a record's lane r + 16 * o
    // holds k-octet o of row r, and a weight chunk's lane c + 16 * o holds
    // k-octet o of column c for both blocks, so octets 2 kh and 2 kh + 1 are
    // two 16-byte reads 256 bytes apart.
    auto run32 = [&](auto ctw_tag, int toff) {
        constexpr int CTW = decltype(ctw_tag)::value;
        constexpr int NG = CTW / 2;
        constexpr bool ODD = (CTW & 1) != 0;
        const int c32 = lane & 31, kh = lane >> 5;
        float sbg[NG], sbo = 0.0f;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            sbg[g] = 0.0f;
            if (SCM == 0) {
                const int t = min(t0 + toff + 2 * g + (c32 >> 4), a.ntiles - 1);
                sbg[g] = reinterpret_cast<const float*>(a.S)[(size_t)t * a.ngrp * 16 + (c32 & 15)];
                asm volatile("" ::"v"(sbg[g]));
            }
        }
        if (ODD && SCM == 0) {
            sbo = reinterpret_cast<const float*>(a.S)[(size_t)min(t0 + toff + CTW - 1, a.ntiles - 1) * a.ngrp * 16 + col];
            asm volatile("" ::"v"(sbo));
        }
        float acc[NG][16], acco[2][4];
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[g][j] = 0.0f;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acco[r][i] = 0.0f;

        // dma_tag: 0 no loads, 1 or 2 the loads of chunk 0 or 1 of the next
        // stage (c_next, at LDS nbase).
        auto compute = [&](const char* cp, auto nb_tag, auto dma_tag, int c_next, uint32_t nbase) {
            constexpr int NB = decltype(nb_tag)::value;
            constexpr bool DMA = decltype(dma_tag)::value != 0;
            constexpr bool FIRST = decltype(dma_tag)::value == 1;
            constexpr int kAhead = 1;            // groups read ahead
            constexpr int NGB = NG * NB;         // group steps
            constexpr int NS = NGB + (ODD ? NB : 0);
            const char* ar = cp + L::kA + 2 * rp * kRecBytes;
            v4i a_h[2], a_l[2];
            float sa[2][16];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                // Two 8-byte halves 256 bytes apart: one ds_read2_b64 into
                // the operand's four registers.
                const char* rb = ar + (c32 >> 4) * kRecBytes + b * 1024 + 16 * ((c32 & 15) + 32 * kh);
                const uint2 h0 = *reinterpret_cast<const uint2*>(rb), h1 = *reinterpret_cast<const uint2*>(rb + 256);
                const uint2 l0 = *reinterpret_cast<const uint2*>(rb + 8), l1 = *reinterpret_cast<const uint2*>(rb + 264);
                a_h[b] = v4i{(int)h0.x, (int)h0.y, (int)h1.x, (int)h1.y};
                a_l[b] = v4i{(int)l0.x, (int)l0.y, (int)l1.x, (int)l1.y};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // rows 8q + 4kh .. +3: record (q >> 1), row 8 (q & 1) + 4 kh
                    const float4 s4 = *reinterpret_cast<const float4*>(ar + (q >> 1) * kRecBytes + kRecA + b * 64 +
                                                                       4 * (8 * (q & 1) + 4 * kh));
                    sa[b][4 * q] = s4.x;
                    sa[b][4 * q + 1] = s4.y;
                    sa[b][4 * q + 2] = s4.z;
                    sa[b][4 * q + 3] = s4.w;
                }
            }
            // The odd tile: 16x16x32 operands, as in the path above, read at
            // the last group step (its registers are free by then).
            uint64_t ah[2][2], al[2][2];
            float so[2][2][4];
            uint4 bwo = make_uint4(0, 0, 0, 0);
            int2 wso = make_int2(0, 0);
            float sbo2[2] = {0.0f, 0.0f};
            auto load_odd = [&]() {
                if (!ODD) return;
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const uint4 q = *reinterpret_cast<const uint4*>(ar + r * kRecBytes + b * 1024 + 16 * lane);
                        ah[r][b] = (uint64_t)q.y << 32 | q.x;
                        al[r][b] = (uint64_t)q.w << 32 | q.z;
                        const float4 s4 = *reinterpret_cast<const float4*>(ar + r * kRecBytes + kRecA + b * 64 + 16 * grp);
                        so[r][b][0] = s4.x;
                        so[r][b][1] = s4.y;
                        so[r][b][2] = s4.z;
                        so[r][b][3] = s4.w;
                    }
                const int t = toff + CTW - 1;
                bwo = *reinterpret_cast<const uint4*>(cp + t * 1024 + 16 * lane);
                if (HP) wso = *reinterpret_cast<const int2*>(cp + L::kWS + t * 128 + 8 * col);
                if (SCM == 2) {
                    const float2 f = *reinterpret_cast<const float2*>(cp + L::kSB + t * 128 + 8 * col);
                    sbo2[0] = f.x;
                    sbo2[1] = f.y;
                } else if (SCM == 1) {
                    sbo2[0] = sbo2[1] = *reinterpret_cast<const float*>(cp + L::kSB + t * 64 + 4 * col);
                } else {
                    sbo2[0] = sbo2[1] = sbo;
                }
            };
            v4i bq[NG][2];  // B operand per group and block
            int2 wsg[NG];
            float sbv[NG][2];
            auto load_group = [&](int g) {
                if (g >= NG) return;
                const int t = toff + 2 * g + (c32 >> 4);
                const char* bp = cp + t * 1024 + 16 * ((c32 & 15) + 32 * kh);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const uint2 lo = *reinterpret_cast<const uint2*>(bp + 8 * b);
                    const uint2 hi = *reinterpret_cast<const uint2*>(bp + 256 + 8 * b);
                    bq[g][b] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
                }
                if (HP) wsg[g] = *reinterpret_cast<const int2*>(cp + L::kWS + t * 128 + 8 * (c32 & 15));
                if (SCM == 2) {
                    const float2 f = *reinterpret_cast<const float2*>(cp + L::kSB + t * 128 + 8 * (c32 & 15));
                    sbv[g][0] = f.x;
                    sbv[g][1] = f.y;
                } else if (SCM == 1) {
                    sbv[g][0] = sbv[g][1] = *reinterpret_cast<const float*>(cp + L::kSB + t * 64 + 4 * (c32 & 15));
                } else {
                    sbv[g][0] = sbv[g][1] = sbg[g];
                }
            };
            auto bop32 = [&](int g, int b) -> v4i { return bq[g][b]; };
            auto bopo = [&](int b) -> uint64_t {
                return b == 0 ? ((uint64_t)bwo.y << 32 | bwo.x) : ((uint64_t)bwo.w << 32 | bwo.z);
            };
            v16i h32[NGB], d32[NGB];
            v4i ho[2][2], dov[2][2];
            const v16i z16 = {};
            auto step_h = [&](int s) {
                if (!HP || s >= NS) return;
                if (s < NGB) {
                    h32[s] = mfma32(a_h[s % NB], bop32(s / NB, s % NB), z16);
                } else {
                    const int b = s - NGB;
#pragma unroll
                    for (int r = 0; r < 2; ++r) ho[b][r] = mfma16(ah[r][b], bopo(b));
                }
            };
            auto step_d = [&](int s) {
                if (s >= NS) return;
                if (s < NGB) {
                    const int g = s / NB, b = s % NB;
                    if (HP) {
                        const int s128 = b == 0 ? wsg[g].x : wsg[g].y;
                        v16i ci;
#pragma unroll
                        for (int j = 0; j < 16; ++j) ci[j] = (h32[s][j] << 8) + s128;
                        d32[s] = mfma32(a_l[b], bop32(g, b), ci);
                    } else {
                        d32[s] = mfma32(a_h[b], bop32(g, b), z16);
                    }
                } else {
                    const int b = s - NGB;
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        if (HP) {
                            const int s128 = b == 0 ? wso.x : wso.y;
                            const v4i ci = {(ho[b][r][0] << 8) + s128, (ho[b][r][1] << 8) + s128,
                                            (ho[b][r][2] << 8) + s128, (ho[b][r][3] << 8) + s128};
                            dov[b][r] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)al[r][b], (long)bopo(b), ci, 0, 0, 0);
                        } else {
                            dov[b][r] = mfma16(ah[r][b], bopo(b));
                        }
                    }
                }
            };
            auto step_e = [&](int s) {
                if (s < NGB) {
                    const int g = s / NB, b = s % NB;
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        acc[g][j] = __builtin_fmaf(sa[b][j], (float)d32[s][j] * sbv[g][b], acc[g][j]);
                } else {
                    const int b = s - NGB;
#pragma unroll
                    for (int r = 0; r < 2; ++r)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acco[r][i] = __builtin_fmaf(so[r][b][i], (float)dov[b][r][i] * sbo2[b], acco[r][i]);
                }
            };
            // Depth-1 pipeline (registers: 16 accumulators per group): step
            // s issues step s+1's h-byte MFMA, runs its own epilogue, which
            // covers that MFMA's latency, then step s+1's shift-add and
            // l-byte MFMA.
#pragma unroll
            for (int g = 0; g < kAhead; ++g) load_group(g);
            if (NGB == 0) load_odd();
            step_h(0);
            step_d(0);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                if (s < NGB && s % NB == 0) load_group(s / NB + kAhead);
                if (s == NGB - 1) load_odd();
                if (DMA && s < kDmaChunk) dma_slot(c_next, nbase, s, FIRST);
                step_h(s + 1);
                step_e(s);
                step_d(s + 1);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (DMA) {
#pragma unroll
                for (int d = NS; d < kDmaChunk; ++d) dma_slot(c_next, nbase, d, FIRST);
            }
        };

        static_assert(kPfChunks == 2, "stage loop");
        constexpr std::integral_constant<int, 2> two{};
        constexpr std::integral_constant<int, 1> one{};
        constexpr std::integral_constant<int, 1> dma0{};
        constexpr std::integral_constant<int, 2> dma1{};
        constexpr std::integral_constant<int, 0> no_dma{};
        issue_stage(0, 0);
        for (int g = 0; g + 1 < nst; ++g) {
            __builtin_amdgcn_s_waitcnt(vm_wait(0));
            lds_barrier();
            if (BITS == 4) {
                expand(g & 1);
                lds_barrier();
            }
            const uint32_t nbase = lds0 + (uint32_t)(((g + 1) & 1) * L::kStage);
            const int cn = (g + 1) * kPfChunks;
            if (active) {
                const char* sp = pf_lds + (g & 1) * L::kStage;
                compute(sp, two, dma0, cn, nbase);
                compute(sp + L::kChunk, two, dma1, min(cn + 1, nch - 1), nbase + (uint32_t)L::kChunk);
            } else {
                issue_stage(g + 1, (g + 1) & 1);
            }
        }
        __builtin_amdgcn_s_waitcnt(vm_wait(0));
        lds_barrier();
        if (BITS == 4) {
            expand((nst - 1) & 1);
            lds_barrier();
        }
        if (!active) return;
        {
            const char* sp = pf_lds + ((nst - 1) & 1) * L::kStage;
            const int c0 = (nst - 1) * kPfChunks;
            if (c0 + 1 < nch) {
                compute(sp, two, no_dma, 0, 0u);
                if (odd) compute(sp + L::kChunk, one, no_dma, 0, 0u);
                else compute(sp + L::kChunk, two, no_dma, 0, 0u);
            } else if (odd) {
                compute(sp, one, no_dma, 0, 0u);
            } else {
                compute(sp, two, no_dma, 0, 0u);
            }
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int tile = t0 + toff + 2 * g + (c32 >> 4);
            if (tile >= a.ntiles) continue;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int m = rt0 * 16 + (j & 3) + 8 * (j >> 2) + 4 * kh;
                if (m < a.M) a.C[(size_t)m * a.N + tile * 16 + (c32 & 15)] = acc[g][j];
            }
        }
        if (ODD) {
            const int tile = t0 + toff + CTW - 1;
            if (tile < a.ntiles) {
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int m = (rt0 + r) * 16 + 4 * grp + i;
                        if (m < a.M) a.C[(size_t)m * a.N + tile * 16 + col] = acco[r][i];
                    }
            }
        }
    };
    if (half == 0) run32(std::integral_constant<int, (CT + 1) / 2>{}, 0);
    else run32(std::integral_constant<int, CT / 2>{}, (CT + 1) / 2);
}

// Activation records for the prefill GEMM: 8 lanes per (row, block) over
// Mpad rows and 2*nch blocks; padding rows and blocks quantize zeros.
template <bool HP>
__global__ __launch_bounds__(256) void quantize_rec_kernel(const float* __restrict__ A, int M, int K, int nblk,
                                                           int nch, int Mpad, uint8_t* __restrict__ R) {
    const int gtid = blockIdx.x * 256 + threadIdx.x;
    const int blk = gtid >> 3, e = gtid & 7;
    const int nb2 = 2 * nch;
    const int m = blk / nb2, j = blk - m * nb2;
    const bool inside = m < Mpad;
    const bool valid = m < M && j < nblk;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v = *reinterpret_cast<const float4*>(A + (size_t)m * K + 32 * j + 4 * e);
    float s;
    int sum;
    uint32_t p0, p1;
    quant8<HP>(v, s, sum, p0, p1);
    if (inside) {
        uint8_t* rec = R + ((size_t)(m >> 4) * nch + (j >> 1)) * kRecBytes;
        const int b = j & 1, r = m & 15;
        uint8_t* p = rec + b * 1024 + ((e >> 1) * 16 + r) * 16 + (e & 1) * 4;
        *reinterpret_cast<uint32_t*>(p) = p0;
        *reinterpret_cast<uint32_t*>(p + 8) = p1;
        if (e == 0) *reinterpret_cast<float*>(rec + kRecA + (b * 16 + r) * 4) = s;
    }
}

// Column tiles per workgroup: the instantiated widths, and the choice that
// minimizes (workgroup rounds) x (tiles per workgroup) at one workgroup per
// CU.  `force` (the BREEZE_HIP_PREFILL_CT environment variable) selects an
// instantiated width instead, for tests and tuning.
constexpr int kPfCts[] = {17, 16, 8, 4};

int pick_pf_ct(int ntiles, int gy, int n_cu, const char* force) {
    if (force) {
        const int v = std::atoi(force);
        for (int ct : kPfCts)
            if (ct == v) return ct;
    }
    int best = kPfCts[0];
    long best_cost = -1;
    for (int ct : kPfCts) {
        const long wgs = (long)((ntiles + ct - 1) / ct) * gy;
        const long cost = (wgs + n_cu - 1) / n_cu * ct;
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = ct;
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
// specials are summed by one thread in element order.  Rows up to kNormStage
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

__device__ inline long long readlane64(long long v, int l) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)v, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)((unsigned long long)v >> 32), l);
    return (long long)((unsigned long long)hi << 32 | lo);
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

template <bool STAGED>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* __restrict__ X, const float* __restrict__ Wt,
                                                                int H, float eps, float* __restrict__ Out) {
    extern __shared__ float norm_row[];                      // STAGED: the row
    __shared__ double spec[kNormMaxSpecial];                 // t, or -(floor(t/u) + 1) for a tie
    __shared__ unsigned long long seg[kNormMaxSpecial + 1];  // sum of k with q specials before
    __shared__ unsigned long long gap[kNormMaxSpecial];      // non-anchor ties after anchor a
    __shared__ int alist[kNormMaxSpecial];                   // special index of anchor a
    __shared__ double wsum_d[kNormThreads / 64];
    __shared__ int wsum_i[kNormThreads / 64];
    __shared__ double ss_s;
    const float* xg = X + (size_t)blockIdx.x * H;
    float* o = Out + (size_t)blockIdx.x * H;
    const int tid = threadIdx.x;
    if (STAGED) {
#pragma unroll 4
        for (int j = tid; j < H; j += kNormThreads) norm_row[j] = xg[j];
        __syncthreads();
    }
    const float* x = STAGED ? norm_row : xg;
    const int per = (H + kNormThreads - 1) / kNormThreads;
    const int j0 = min(tid * per, H), j1 = min(j0 + per, H);

    // STAGED: this thread's terms (0 past its range) and, after the
    // classification, their k and which of them are specials / ties.
    double tv[STAGED ? kNormPer : 1];
    unsigned long long kv[STAGED ? kNormPer : 1];
    unsigned smask = 0, tmask = 0;
    double loc = 0.0;
    int nan = 0, inf = 0;
    if constexpr (STAGED) {
#pragma unroll
        for (int i = 0; i < kNormPer; ++i) {
            const int j = j0 + i;
            const float xv = j < j1 ? x[j] : 0.0f;
            tv[i] = (double)xv * (double)xv;
            nan |= tv[i] != tv[i];
            inf |= tv[i] == __builtin_inf();
            loc += tv[i];
        }
    } else {
        for (int j = j0; j < j1; ++j) {
            const double t = (double)x[j] * (double)x[j];
            nan |= t != t;
            inf |= t == __builtin_inf();
            loc += t;
        }
    }
    const int any_nan = __syncthreads_or(nan), any_inf = __syncthreads_or(inf);
    if (any_nan || any_inf) {
        if (tid == 0) ss_s = any_nan ? __builtin_nan("") : __builtin_inf();
    } else {
        double tot_d;
        const double base = block_exclusive_scan<double>(loc, wsum_d, &tot_d);
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
        } else if (tid == 0) {
            double acc = 0.0;
            for (int j = 0; j < H; ++j) acc += (double)x[j] * (double)x[j];
            ss_s = acc;
        }
    }
    __syncthreads();
    const float inv = 1.0f / sqrtf((float)(ss_s / (double)H) + eps);
#pragma unroll 4
    for (int j = tid; j < H; j += kNormThreads) o[j] = x[j] * inv * Wt[j];
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

// part [nparts][M] -> out[m].
// u = silu(g) * u elementwise, silu(x) = x / (1 + exp(-x)) as in
// kernel/qwen35_decoder.cpp:129 and 408; the same expression as the paired
// decode kernel's epilogue, so both paths give the same bits.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ g, float* __restrict__ u,
                                                       size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float x = g[i];
        u[i] = x / (1.0f + expf(-x)) * u[i];
    }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const unsigned long long* __restrict__ part,
                                                           int nparts, int M, int64_t* __restrict__ out) {
    const int m = blockIdx.x;
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < nparts; i += 256) best = max(best, part[(size_t)i * M + m]);
    best = block_max_key(best);
    if (threadIdx.x == 0) out[m] = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
}

// ------------------------------------------------------------------ workspace

struct Workspace {
    std::mutex mu;
    uint8_t* aq = nullptr;
    float* sa = nullptr;
    int* sq = nullptr;
    size_t rows_cap = 0, nblk4_cap = 0;
    unsigned long long* parts = nullptr;
    unsigned int* ticket = nullptr;  // decode argmax: ticket counter, then 8 row keys; zero between calls
    size_t parts_cap = 0;
    uint8_t* rec = nullptr;  // prefill activation records
    size_t rec_cap = 0;
    bool pf_attr[64] = {};
    float* gate = nullptr;  // gate projection of the unpaired gate/up path
    size_t gate_cap = 0;
    float* hA = nullptr;  // device staging for the host-pointer entry points
    float* hC = nullptr;
    size_t hA_cap = 0, hC_cap = 0;
    hipStream_t stream = nullptr;
    int n_cu = 0;
    bool attr_set[128] = {};
};

constexpr int kMaxDevices = 64;
Workspace g_ws[kMaxDevices];

template <typename T>
bool grow(T** p, size_t* cap, size_t need, const char* what) {
    if (need <= *cap) return true;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    if (!hip_ok(hipMalloc(reinterpret_cast<void**>(p), need * sizeof(T)), what)) return false;
    *cap = need;
    return true;
}

bool ensure_quant(Workspace& w, size_t rows, size_t nblk4) {
    if (rows * nblk4 <= w.rows_cap * w.nblk4_cap && nblk4 <= w.nblk4_cap && rows <= w.rows_cap &&
        w.aq)
        return true;
    const size_t r = std::max(rows, w.rows_cap), nb = std::max(nblk4, w.nblk4_cap);
    size_t c1 = 0, c2 = 0, c3 = 0;
    if (w.aq) (void)hipFree(w.aq);
    if (w.sa) (void)hipFree(w.sa);
    if (w.sq) (void)hipFree(w.sq);
    w.aq = nullptr;
    w.sa = nullptr;
    w.sq = nullptr;
    w.rows_cap = w.nblk4_cap = 0;
    if (!grow(&w.aq, &c1, r * nb * 64, "workspace alloc") || !grow(&w.sa, &c2, r * nb, "workspace alloc") ||
        !grow(&w.sq, &c3, r * nb, "workspace alloc"))
        return false;
    w.rows_cap = r;
    w.nblk4_cap = nb;
    return true;
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

constexpr int kLdsMax = 160 * 1024;
constexpr int kFusedMaxBlocks = kQuantPasses * 128;  // row-blocks the prologue quantizes

// LDS bytes of the decode kernel, or 0 if the activation records of a row
// group do not fit (in LDS, or in the prologue's 6-uint4-per-thread record
// copy).
int plan_dec_lds(const GemvArgs& a, int Mr_max, int JG, bool p64 = false) {
    if (Mr_max * a.nblk > kFusedMaxBlocks && Mr_max * a.nblk * 4 > 6 * kDecWaves * 64) return 0;
    const int total = dec_lds(Mr_max, a.nblk, JG, p64).total;
    return total <= kLdsMax ? total : 0;
}

template <int BITS, bool HP, bool FUSED, bool EXTRA, int R, bool PAIR, bool P64>
hipError_t launch_dec_t(Workspace& w, const GemvArgs& a, int grid, int lds, hipStream_t st) {
    auto kern = dec_kernel<BITS, HP, FUSED, EXTRA, R, PAIR, P64>;
    const int key = (BITS == 8 ? 1 : 0) | (HP ? 2 : 0) | (FUSED ? 4 : 0) | (EXTRA ? 8 : 0) | ((R / 2 - 1) << 4) |
                    (PAIR ? 32 : 0) | (P64 ? 64 : 0);
    if (!w.attr_set[key]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
        if (e != hipSuccess) return e;
        w.attr_set[key] = true;
    }
    const void* act = FUSED ? static_cast<const void*>(a.A) : static_cast<const void*>(a.Aq);
    const int npw = (a.nbg + kProducers - 1) / kProducers;
    const int misc = a.sc_shift | a.RG << 8 | a.pair_xcd << 10 | npw << 16;
    const int base_t = a.ntiles / a.NG, rem_t = a.ntiles - base_t * a.NG;
    kern<<<grid, kDecWaves * 64, lds, st>>>(act, a.W, a.S, base_t, a.nblk, a.M, a.nbg, rem_t, a.NG, a.ngrp, misc, a);
    return hipGetLastError();
}

// Ring depth R (weight units in flight per wave).  Two units per producer
// (30 KB per CU) measured fastest on every decode workload: deeper rings
// put more requests in flight than the memory system turns into bandwidth.
constexpr int kDecRing = 2;

template <int BITS, bool HP, bool FUSED, bool EXTRA>
hipError_t launch_dec_r(Workspace& w, const GemvArgs& a, int grid, int lds, bool pair, bool p64,
                        hipStream_t st) {
    if (p64) return pair ? launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, true, true>(w, a, grid, lds, st)
                         : launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, false, true>(w, a, grid, lds, st);
    return pair ? launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, true, false>(w, a, grid, lds, st)
                : launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, false, false>(w, a, grid, lds, st);
}

template <int BITS, bool HP>
hipError_t launch_dec_bits(Workspace& w, const GemvArgs& a, int grid, int lds, bool pair, bool p64, bool fused,
                           bool extra, hipStream_t st) {
    if (extra) return fused ? launch_dec_r<BITS, HP, true, true>(w, a, grid, lds, pair, p64, st)
                            : launch_dec_r<BITS, HP, false, true>(w, a, grid, lds, pair, p64, st);
    return fused ? launch_dec_r<BITS, HP, true, false>(w, a, grid, lds, pair, p64, st)
                 : launch_dec_r<BITS, HP, false, false>(w, a, grid, lds, pair, p64, st);
}

template <int BITS, bool HP>
hipError_t launch_rows_bits(const GemvArgs& a, dim3 grid, bool dots, hipStream_t st) {
    if (dots) rows_kernel<BITS, HP, true><<<grid, kRowWaves * 64, 0, st>>>(a);
    else rows_kernel<BITS, HP, false><<<grid, kRowWaves * 64, 0, st>>>(a);
    return hipGetLastError();
}

template <int BITS, bool HP, int SCM, int CT>
hipError_t launch_pf_t(Workspace& w, const PfArgs& p, dim3 grid, hipStream_t st) {
    using L = PfLayout<CT, SCM, BITS>;
    auto kern = prefill_kernel<BITS, HP, SCM, CT>;
    int slot = 0;
    while (kPfCts[slot] != CT) ++slot;
    const int key = (HP ? 1 : 0) | SCM << 1 | slot << 3 | (BITS == 4 ? 32 : 0);
    if (!w.pf_attr[key]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
        if (e != hipSuccess) return e;
        w.pf_attr[key] = true;
    }
    kern<<<grid, kPfWaves * 64, L::kBytes, st>>>(p);
    return hipGetLastError();
}

template <int BITS, bool HP, int SCM>
hipError_t launch_pf_scm(Workspace& w, const PfArgs& p, int ct, dim3 grid, hipStream_t st) {
    switch (ct) {
        case 17: return launch_pf_t<BITS, HP, SCM, 17>(w, p, grid, st);
        case 16: return launch_pf_t<BITS, HP, SCM, 16>(w, p, grid, st);
        case 8: return launch_pf_t<BITS, HP, SCM, 8>(w, p, grid, st);
        default: return launch_pf_t<BITS, HP, SCM, 4>(w, p, grid, st);
    }
}

template <int BITS, bool HP>
hipError_t launch_pf(Workspace& w, const PfArgs& p, int scm, int ct, dim3 grid, hipStream_t st) {
    if (scm == 2) return launch_pf_scm<BITS, HP, 2>(w, p, ct, grid, st);
    if (scm == 1) return launch_pf_scm<BITS, HP, 1>(w, p, ct, grid, st);
    return launch_pf_scm<BITS, HP, 0>(w, p, ct, grid, st);
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

// Quantize + block dots + epilogue for M rows on `st`.  Exactly one of
// dC / dCs is non-null; dIdx (optional) receives the per-row argmax.
constexpr int kNotPairable = -100;  // run() with h2: the decode kernel does not take this call

// Gate and up handles the paired decode kernel can stream together: the same
// device, shape and device layout.
bool same_layout(const Handle* a, const Handle* b) {
    return a->device == b->device && a->N == b->N && a->K == b->K && a->bits == b->bits && a->nbg == b->nbg &&
           a->sc_shift == b->sc_shift && a->ngrp == b->ngrp && a->sc_blk == b->sc_blk && a->extra == b->extra &&
           (a->Z == nullptr) == (b->Z == nullptr) && (a->D == nullptr) == (b->D == nullptr);
}

// h2 (gate/up pairing): a second handle with the same layout (same_layout).
// Returns kNotPairable, having launched nothing, when the decode kernel does
// not take the call.
int run(Handle* h, const float* dA, int M, float* dC, int32_t* dCs, int64_t* dIdx, hipStream_t st,
        const Handle* h2 = nullptr) {
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
    Workspace& w = g_ws[dev];
    const bool hp = g_hi_prec != 0;
    const bool dots = dCs != nullptr;
    const int JG = h->bits == 8 ? 2 : 4;

    GemvArgs a{};
    fill_args(h, a, M);
    a.A = dA;
    a.C = dC;
    a.Cs = dCs;

    // Decode kernel for M <= 8 (one or two row groups of 4); the rows kernel
    // serves larger M, the block-integer export and shapes whose activation
    // records do not fit in LDS.  The decode kernel quantizes small
    // activations itself; larger ones go through the stand-alone quantizer
    // once instead of once per workgroup.
    const int Mr_max = std::min(M, 4);
    // One or two rows: block pairs per MFMA (P64) when its larger record
    // layout fits in LDS.
    const int lds_p64 = (M <= 2 && !dots) ? plan_dec_lds(a, Mr_max, JG, true) : 0;
    const bool p64 = lds_p64 > 0;
    const int lds = p64 ? lds_p64 : (M <= 8 && !dots) ? plan_dec_lds(a, Mr_max, JG) : 0;
    const bool dec = lds > 0;
    if (h2 && !dec) return kNotPairable;
    const bool fused = dec && Mr_max * h->nblk <= kFusedMaxBlocks;
    // Prefill GEMM: more than 8 rows without a legacy corr.
    const bool pre = !dec && !dots && M > 8 && (h->bits == 4 || h->WS) && !h->has_dl;
    const int Mpad = (M + kPfRows - 1) / kPfRows * kPfRows;
    const int nch_rec = (h->nblk + 1) / 2;  // record chunks of two blocks
    if (pre) {
        // Records in MFMA operand order for the prefill GEMM.
        if (!grow(&w.rec, &w.rec_cap, (size_t)(Mpad / 16) * nch_rec * kRecBytes, "workspace alloc")) return -4;
        const size_t threads = (size_t)Mpad * nch_rec * 2 * 8;
        const unsigned qb = (unsigned)((threads + 255) / 256);
        if (hp) quantize_rec_kernel<true><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, nch_rec, Mpad, w.rec);
        else quantize_rec_kernel<false><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, nch_rec, Mpad, w.rec);
        if (!hip_ok(hipGetLastError(), "quantize launch")) return -5;
    } else if (!fused) {
        if (!ensure_quant(w, M, h->nblk4)) return -4;
        const size_t threads = (size_t)M * h->nblk * 8;
        const unsigned qb = (unsigned)((threads + 255) / 256);
        if (hp) quantize_kernel<true><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, h->nblk4, w.aq, w.sa, w.sq);
        else quantize_kernel<false><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, h->nblk4, w.aq, w.sa, w.sq);
        if (!hip_ok(hipGetLastError(), "quantize launch")) return -5;
        a.Aq = w.aq;
        a.Sa = w.sa;
        a.Sq = w.sq;
    }

    hipError_t e;
    if (dec) {
        const int n_cu = device_cus(w, dev);
        a.RG = (M + 3) / 4;
        if (a.RG == 1) {
            a.NG = std::min(a.ntiles, n_cu);
            a.pair_xcd = 0;
        } else {
            const int ng = std::min(a.ntiles, std::max(1, n_cu / 2));
            a.pair_xcd = ng % 8 == 0 ? 1 : 0;
            a.NG = ng;
        }
        const bool pair = h2 != nullptr;
        if (pair) {
            a.W2 = h2->W;
            a.S2 = h2->S;
            a.Z2 = h2->Z;
            a.D2 = h2->D;
        }
        if (dIdx) {
            if (!w.ticket) {
                // Allocated and zeroed once per device (not under graph capture);
                // the kernel's last workgroup re-arms it to zero.
                if (!hip_ok(hipMalloc(&w.ticket, 9 * sizeof(unsigned long long)), "argmax workspace")) return -4;
                if (!hip_ok(hipMemset(w.ticket, 0, 9 * sizeof(unsigned long long)), "argmax workspace")) {
                    (void)hipFree(w.ticket);
                    w.ticket = nullptr;
                    return -4;
                }
            }
            a.ticket = w.ticket;
            a.key = reinterpret_cast<unsigned long long*>(w.ticket) + 1;
            a.idx = dIdx;
        }
        const int grid = a.NG * a.RG;
        const bool x = h->extra;
        if (h->bits == 8) e = hp ? launch_dec_bits<8, true>(w, a, grid, lds, pair, p64, fused, x, st)
                                 : launch_dec_bits<8, false>(w, a, grid, lds, pair, p64, fused, x, st);
        else e = hp ? launch_dec_bits<4, true>(w, a, grid, lds, pair, p64, fused, x, st)
                    : launch_dec_bits<4, false>(w, a, grid, lds, pair, p64, fused, x, st);
    } else if (pre) {
        PfArgs p{};
        p.W = reinterpret_cast<const char*>(h->W);
        p.WS = reinterpret_cast<const char*>(h->WS);
        p.S = reinterpret_cast<const char*>(h->S);
        p.Z = reinterpret_cast<const char*>(h->Z);
        p.R = reinterpret_cast<const char*>(w.rec);
        p.C = dC;
        p.M = M;
        p.N = h->N;
        p.nblk = h->nblk;
        p.nch = nch_rec;
        p.ngrp = h->ngrp;
        p.sc_shift = h->sc_shift;
        p.ntiles = h->N / 16;
        p.nbg = h->nbg;
        const int scm = h->sc_blk ? 2 : (h->sc_shift == 31 ? 0 : 1);
        if (h->bits == 4 && scm == 2 && !h->Z) {
            set_err("internal: INT4 handle with per-block scales has no zero points");
            return -5;
        }
        const int gy = Mpad / kPfRows;
        const int ct = pick_pf_ct(p.ntiles, gy, device_cus(w, dev), std::getenv("BREEZE_HIP_PREFILL_CT"));
        const dim3 grid((unsigned)((p.ntiles + ct - 1) / ct), (unsigned)gy);
        if (h->bits == 8) e = hp ? launch_pf<8, true>(w, p, scm, ct, grid, st) : launch_pf<8, false>(w, p, scm, ct, grid, st);
        else e = hp ? launch_pf<4, true>(w, p, scm, ct, grid, st) : launch_pf<4, false>(w, p, scm, ct, grid, st);
        e = hipGetLastError();
    } else {
        const dim3 grid(a.ntiles, (M + kRowsPerWG - 1) / kRowsPerWG);
        if (h->bits == 8) e = hp ? launch_rows_bits<8, true>(a, grid, dots, st)
                                 : launch_rows_bits<8, false>(a, grid, dots, st);
        else e = hp ? launch_rows_bits<4, true>(a, grid, dots, st) : launch_rows_bits<4, false>(a, grid, dots, st);
    }
    if (!hip_ok(e, "matmul launch")) return -5;

    if (dIdx && !dots && !dec) {
        // The decode kernel merges its own argmax (last workgroup).
        const int nparts = (h->N + kArgmaxChunk - 1) / kArgmaxChunk;
        if (!grow(&w.parts, &w.parts_cap, (size_t)M * nparts, "argmax workspace")) return -4;
        argmax_partial_kernel<<<dim3(nparts, M), 256, 0, st>>>(dC, h->N, w.parts);
        argmax_final_kernel<<<M, 256, 0, st>>>(w.parts, nparts, M, dIdx);
        if (!hip_ok(hipGetLastError(), "argmax launch")) return -5;
    }
    return 0;
}

bool check_dims(int N, int K, int bits) {
    if (N <= 0 || K <= 0 || N % 16 || K % 32 || (bits != 4 && bits != 8)) {
        set_err("contract violation: need N>0, K>0, N%%16==0, K%%32==0, bits in {4,8} "
                "(got N=%d K=%d bits=%d)", N, K, bits);
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
    if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&dec_kernel<8, true, true, false, kDecRing, false, false>)) !=
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
    return run(h, dA, M, dC, nullptr, nullptr, static_cast<hipStream_t>(stream));
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
    if (same_layout(hg, hu)) {
        const int rc = run(hg, dA, M, dC, nullptr, nullptr, st, hu);
        if (rc != kNotPairable) return rc;
    }
    // Two projections, then the elementwise epilogue.
    if (M <= 0 || !dC) return run(hu, dA, M, dC, nullptr, nullptr, st);
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != hg->device) {
        set_err("handle lives on device %d but device %d is current", hg->device, dev);
        return -3;
    }
    Workspace& w = g_ws[dev];
    const size_t n = (size_t)M * hg->N;
    if (!grow(&w.gate, &w.gate_cap, n, "workspace alloc")) return -4;
    int rc = run(hg, dA, M, w.gate, nullptr, nullptr, st);
    if (rc == 0) rc = run(hu, dA, M, dC, nullptr, nullptr, st);
    if (rc) return rc;
    silu_mul_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(w.gate, dC, n);
    return hip_ok(hipGetLastError(), "silu-mul launch") ? 0 : -5;
}

int i4_matmul_argmax_dev(void* handle, const float* dA, int M, float* dC, int64_t* dIdx, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    if (!dIdx) {
        set_err("null argmax output");
        return -2;
    }
    return run(h, dA, M, dC, nullptr, dIdx, static_cast<hipStream_t>(stream));
}

int i4_block_dots_dev(void* handle, const float* dA, int M, int32_t* dCs, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    return run(h, dA, M, nullptr, dCs, nullptr, static_cast<hipStream_t>(stream));
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
    Workspace& w = g_ws[h->device];
    std::lock_guard<std::mutex> lock(w.mu);
    if (!w.stream && !hip_ok(hipStreamCreateWithFlags(&w.stream, hipStreamNonBlocking), "stream")) return;
    const size_t na = (size_t)M * h->K, nc = (size_t)M * h->N;
    if (!grow(&w.hA, &w.hA_cap, na, "staging alloc") || !grow(&w.hC, &w.hC_cap, nc, "staging alloc")) return;
    if (!hip_ok(hipMemcpyAsync(w.hA, A, na * 4, hipMemcpyHostToDevice, w.stream), "upload A")) return;
    if (run(h, w.hA, M, w.hC, nullptr, nullptr, w.stream) != 0) {
        (void)hipStreamSynchronize(w.stream);
        return;
    }
    if (!hip_ok(hipMemcpyAsync(C, w.hC, nc * 4, hipMemcpyDeviceToHost, w.stream), "download C")) return;
    (void)hip_ok(hipStreamSynchronize(w.stream), "matmul");
    if (cur != h->device) (void)hipSetDevice(cur);
}

void i4_matmul_region(void* handle, const float* A, int M, float* C, uint8_t*, float*) {
    i4_matmul(handle, A, M, C);
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
    if (M < 0 || H <= 0) {
        set_err("need M >= 0 and H > 0 (got M %d, H %d)", M, H);
        return -1;
    }
    if (M == 0) return 0;
    if (!dX || !dW || !dOut) {
        set_err("null device pointer");
        return -2;
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (H <= kNormStage)
        rmsnorm_kernel<true><<<(unsigned)M, kNormThreads, (size_t)H * sizeof(float), st>>>(dX, dW, H, eps, dOut);
    else
        rmsnorm_kernel<false><<<(unsigned)M, kNormThreads, 0, st>>>(dX, dW, H, eps, dOut);
    return hip_ok(hipGetLastError(), "rmsnorm launch") ? 0 : -3;
}

}  // extern "C"

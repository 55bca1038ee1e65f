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
//   * The FP32 chain is evaluated in block order per (m, n): waves compute
//     f = f32(cs)*scale for a segment of blocks into LDS, then one lane per
//     (m, n) folds the segment into its accumulator.  Bit-identical to the
//     reference for every M, so row m of an M-row call equals a 1-row call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
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

// ------------------------------------------------------------------ layout constants

// Position p of an 8-byte MFMA operand holds k = 8*octet + kPerm8[p]: the
// order in which the INT4 unpack (low nibbles, then high nibbles of four
// packed bytes) delivers weights.  INT8 weights and the activations use the
// same order, so A and B always agree on k.
constexpr int kPerm8[8] = {0, 2, 4, 6, 1, 3, 5, 7};

constexpr int kWaves = 4;          // waves per workgroup
constexpr int kChunksPerWave = 2;  // 16-byte weight chunks per wave per segment
constexpr int kRowsPerWG = 8;      // activation rows per workgroup (two MFMA row groups)

constexpr uint32_t kMagic = 0xB2EE2E51u;

struct Handle {
    uint32_t magic;
    int N, K, nblk, bits;  // bits of the device representation
    int nbg;               // 16-byte chunks per column tile along K
    int sc_shift, ngrp, sc_group;
    bool has_zp, has_dl;
    int device;
    uint4* W;    // [N/16][nbg][64 lanes] 16-byte chunks
    float* S;    // [N][ngrp]
    int8_t* Z;   // [N][nblk] zero points, INT4 only, NULL = all 8
    int32_t* D;  // [N][nblk] legacy corr delta, NULL = none
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

// ------------------------------------------------------------------ kernels

// MatMulNBits bytes -> 16-byte lane chunks.  Chunk (t, cg) of a 16-column
// tile is 64 lanes x 16 bytes; lane l serves column 16t + (l & 15) and
// k-octet (l >> 4) of each block, i.e. exactly the B operand of
// v_mfma_i32_16x16x32_i8.  INT8: 2 blocks per chunk, bytes kPerm8-ordered
// and xor 0x80.  INT4: 4 blocks per chunk, the octet's 4 packed bytes as is.
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
        const uint8_t x = raw_signed ? 0 : 0x80;
        for (int hb = 0; hb < 2; ++hb) {
            const int j = cg * 2 + hb;
            if (j >= nblk) continue;
            const uint8_t* src = raw + ((size_t)n * nblk + j) * 32 + oct * 8;
            uint32_t lo = 0, hi = 0;
            for (int p = 0; p < 4; ++p) lo |= (uint32_t)(uint8_t)(src[kPerm8[p]] ^ x) << (8 * p);
            for (int p = 4; p < 8; ++p) hi |= (uint32_t)(uint8_t)(src[kPerm8[p]] ^ x) << (8 * (p - 4));
            w[2 * hb] = lo;
            w[2 * hb + 1] = hi;
        }
    } else {
        for (int q = 0; q < 4; ++q) {
            const int j = cg * 4 + q;
            if (j >= nblk) continue;
            const uint8_t* src = raw + ((size_t)n * nblk + j) * 16 + oct * 4;
            w[q] = (uint32_t)src[0] | (uint32_t)src[1] << 8 | (uint32_t)src[2] << 16 |
                   (uint32_t)src[3] << 24;
        }
    }
    out[o] = make_uint4(w[0], w[1], w[2], w[3]);
}

// Activation quantization, one thread per (row, 32-block).  Writes the
// 64-byte record [part 0: 32 bytes][part 1: 32 bytes], each kPerm8-ordered
// per octet: INT16 mode part 0 = h, part 1 = l (signed halves); INT8 mode
// part 0 = q, part 1 = 0.  Also the block scale s and sum(q).
template <bool HP>
__global__ void quantize_kernel(const float* __restrict__ A, int M, int K, int nblk,
                                uint4* __restrict__ Aq, float* __restrict__ Sa,
                                int* __restrict__ Sq) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= M * nblk) return;
    const int m = idx / nblk, j = idx - m * nblk;
    const float4* src = reinterpret_cast<const float4*>(A + (size_t)m * K + 32 * j);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 x = src[i];
        v[4 * i] = x.x;
        v[4 * i + 1] = x.y;
        v[4 * i + 2] = x.z;
        v[4 * i + 3] = x.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float a = fabsf(v[i]);
        amax = a > amax ? a : amax;
    }
    constexpr int qmax = HP ? 32767 : 127;
    const float s = amax / (float)qmax;
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    int sum = 0;
    uint8_t p0[32], p1[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float prod = v[i] * inv;
        int q = 0;
        if (__builtin_isfinite(prod)) {
            q = (int)rintf(prod);
            q = q > qmax ? qmax : (q < -qmax ? -qmax : q);
        }
        sum += q;
        if (HP) {
            const unsigned u = (unsigned)(q + 32768);
            p0[i] = (uint8_t)((u >> 8) ^ 0x80u);
            p1[i] = (uint8_t)((u & 0xFFu) ^ 0x80u);
        } else {
            p0[i] = (uint8_t)(int8_t)q;
            p1[i] = 0;
        }
    }
    uint32_t w[16];
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
        for (int oct = 0; oct < 4; ++oct)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                uint32_t x = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int k = oct * 8 + kPerm8[half * 4 + b];
                    x |= (uint32_t)(part ? p1[k] : p0[k]) << (8 * b);
                }
                w[part * 8 + oct * 2 + half] = x;
            }
    uint4* dst = Aq + (size_t)idx * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    Sa[idx] = s;
    Sq[idx] = sum;
}

struct QmmArgs {
    const uint4* W;
    const float* S;
    const int8_t* Z;
    const int32_t* D;
    const uint2* Aq;   // [M][nblk][8] 8-byte operand pieces
    const float* Sa;   // [M][nblk]
    const int* Sq;     // [M][nblk]
    float* C;          // [M][N]
    int32_t* Cs;       // [M][N][nblk] (block-dot export only)
    int M, N, nblk, nbg, sc_shift, ngrp;
};

template <int BITS, bool HP, bool HAS_ZP, bool HAS_DL, bool DOTS>
__global__ __launch_bounds__(kWaves * 64) void qmm_kernel(QmmArgs a) {
    constexpr int JG = BITS == 8 ? 2 : 4;  // blocks per 16-byte chunk
    constexpr int SEG = kWaves * kChunksPerWave * JG;
    __shared__ float fbuf[kRowsPerWG][SEG][16];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x;
    const int m0 = blockIdx.y * kRowsPerWG;
    const int Mc = min(kRowsPerWG, a.M - m0);
    const int nmf = (Mc + 3) >> 2;
    // MFMA lane roles: B column / output column, k-octet / output row group.
    const int col = lane & 15, grp = lane >> 4;
    const int arow = lane & 15, arg = arow >> 2, ars = arow & 3;
    const int n = t * 16 + col;
    // Chain role of this thread in phase 2.
    const int cm = threadIdx.x >> 4, ccol = threadIdx.x & 15;
    float acc = 0.0f;

    const int nseg = (a.nblk + SEG - 1) / SEG;
    for (int s = 0; s < nseg; ++s) {
        const int j0 = s * SEG;
#pragma unroll
        for (int c = 0; c < kChunksPerWave; ++c) {
            const int cg = j0 / JG + wave * kChunksPerWave + c;
            if (cg * JG >= a.nblk) break;
            const uint4 wv = a.W[((size_t)t * a.nbg + cg) * 64 + lane];
#pragma unroll
            for (int jb = 0; jb < JG; ++jb) {
                const int j = cg * JG + jb;
                if (j >= a.nblk) break;
                uint64_t bop;
                if (BITS == 8) {
                    const uint32_t lo = jb == 0 ? wv.x : wv.z, hi = jb == 0 ? wv.y : wv.w;
                    bop = (uint64_t)hi << 32 | lo;
                } else {
                    const uint32_t w = jb == 0 ? wv.x : jb == 1 ? wv.y : jb == 2 ? wv.z : wv.w;
                    bop = (uint64_t)((w >> 4) & 0x0F0F0F0Fu) << 32 | (w & 0x0F0F0F0Fu);
                }
                for (int mi = 0; mi < nmf; ++mi) {
                    const int ml = mi * 4 + arg;
                    uint64_t aop = 0;
                    if (ars == 2) {
                        aop = 0x0101010101010101ull;
                    } else if (ars < 2 && ml < Mc) {
                        const uint2 x = a.Aq[((size_t)(m0 + ml) * a.nblk + j) * 8 + ars * 4 + grp];
                        aop = (uint64_t)x.y << 32 | x.x;
                    }
                    const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)aop, (long)bop,
                                                                        v4i{0, 0, 0, 0}, 0, 0, 0);
                    const int me = mi * 4 + grp;
                    if (me < Mc) {
                        const size_t row = (size_t)(m0 + me);
                        int cs = HP ? d[0] * 256 + d[1] + d[2] * 128 : d[0];
                        if (BITS == 4) {
                            const int zp = HAS_ZP ? (int)a.Z[(size_t)n * a.nblk + j] : 8;
                            cs -= zp * a.Sq[row * a.nblk + j];
                        }
                        if (HAS_DL) cs += (HP ? 256 : 1) * a.D[(size_t)n * a.nblk + j];
                        if (DOTS) {
                            a.Cs[(row * a.N + n) * a.nblk + j] = cs;
                        } else {
                            fbuf[me][j - j0][col] =
                                (float)cs * a.S[(size_t)n * a.ngrp + (j >> a.sc_shift)];
                        }
                    }
                }
            }
        }
        if (!DOTS) {
            __syncthreads();
            if (cm < Mc) {
                const int jn = min(SEG, a.nblk - j0);
                const float* sa = a.Sa + (size_t)(m0 + cm) * a.nblk + j0;
                for (int jj = 0; jj < jn; ++jj) acc = __builtin_fmaf(sa[jj], fbuf[cm][jj][ccol], acc);
            }
            __syncthreads();
        }
    }
    if (!DOTS && cm < Mc) a.C[(size_t)(m0 + cm) * a.N + t * 16 + ccol] = acc;
}

// First-maximum argmax per row with numpy.argmax semantics.  Keys order by
// value (NaN highest, -0 == +0) and then by lower index.
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

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ C, int N,
                                                             unsigned long long* __restrict__ part) {
    const int m = blockIdx.y, c = blockIdx.x;
    const int lo = c * kArgmaxChunk, hi = min(N, lo + kArgmaxChunk);
    unsigned long long best = 0;
    for (int i = lo + (int)threadIdx.x; i < hi; i += 256)
        best = max(best, argmax_key(C[(size_t)m * N + i], i));
    best = block_max_key(best);
    if (threadIdx.x == 0) part[(size_t)m * gridDim.x + c] = best;
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const unsigned long long* __restrict__ part,
                                                           int nparts, int64_t* __restrict__ out) {
    const int m = blockIdx.x;
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < nparts; i += 256) best = max(best, part[(size_t)m * nparts + i]);
    best = block_max_key(best);
    if (threadIdx.x == 0) out[m] = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
}

// ------------------------------------------------------------------ workspace

struct Workspace {
    std::mutex mu;
    uint4* aq = nullptr;
    float* sa = nullptr;
    int* sq = nullptr;
    size_t blocks_cap = 0;  // rows * nblk capacity
    unsigned long long* parts = nullptr;
    size_t parts_cap = 0;
    float* hA = nullptr;  // device staging for the host-pointer entry points
    float* hC = nullptr;
    size_t hA_cap = 0, hC_cap = 0;
    hipStream_t stream = nullptr;
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

bool ensure_blocks(Workspace& w, size_t rows_blocks) {
    if (rows_blocks <= w.blocks_cap) return true;
    size_t cap = 0;
    bool ok = grow(&w.aq, &cap, rows_blocks * 4, "workspace alloc");
    cap = 0;
    ok = ok && grow(&w.sa, &cap, rows_blocks, "workspace alloc");
    cap = 0;
    ok = ok && grow(&w.sq, &cap, rows_blocks, "workspace alloc");
    w.blocks_cap = ok ? rows_blocks : 0;
    return ok;
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
//   raw: MatMulNBits bytes [N][nblk][16 or 32] (INT8 either unsigned w+128 or,
//        with raw_signed, already signed w); scales fp32 [N][nblk];
//   zp:  INT4 zero points [N][nblk] or empty; delta: legacy [N][nblk] or empty.
void* build_handle(const uint8_t* raw, bool raw_signed, const float* scales, int N, int K,
                   int bits, const std::vector<int8_t>& zp, const std::vector<int32_t>& delta) {
    const int nblk = K / 32;
    const int JG = bits == 8 ? 2 : 4;
    const int nbg = (nblk + JG - 1) / JG;

    // Repeated scales are stored once: per column, or per aligned group of
    // 2^k blocks (bitwise comparison, so any value is kept as given).
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
    std::vector<float> sc_compact((size_t)N * ngrp);
    for (int n = 0; n < N; ++n)
        for (int g = 0; g < ngrp; ++g)
            sc_compact[(size_t)n * ngrp + g] =
                scales[(size_t)n * nblk + (sc_shift == 31 ? 0 : (g << sc_shift))];

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
    h->sc_shift = sc_shift;
    h->ngrp = ngrp;
    h->sc_group = sc_group;
    h->has_zp = !zp.empty();
    h->has_dl = !delta.empty();
    (void)hipGetDevice(&h->device);

    const size_t wbytes = (size_t)(N / 16) * nbg * 64 * 16;
    const size_t rawbytes = (size_t)N * nblk * 4 * bits;
    uint8_t* draw = nullptr;
    bool ok = hip_ok(hipMalloc(&h->W, wbytes), "weight alloc") &&
              hip_ok(hipMalloc(&h->S, sc_compact.size() * 4), "scale alloc") &&
              (!h->has_zp || hip_ok(hipMalloc(&h->Z, zp.size()), "zero-point alloc")) &&
              (!h->has_dl || hip_ok(hipMalloc(&h->D, delta.size() * 4), "corr alloc")) &&
              hip_ok(hipMalloc(&draw, rawbytes), "staging alloc");
    ok = ok && hip_ok(hipMemcpy(draw, raw, rawbytes, hipMemcpyHostToDevice), "weight upload") &&
         hip_ok(hipMemcpy(h->S, sc_compact.data(), sc_compact.size() * 4, hipMemcpyHostToDevice),
                "scale upload") &&
         (!h->has_zp || hip_ok(hipMemcpy(h->Z, zp.data(), zp.size(), hipMemcpyHostToDevice),
                               "zero-point upload")) &&
         (!h->has_dl || hip_ok(hipMemcpy(h->D, delta.data(), delta.size() * 4, hipMemcpyHostToDevice),
                               "corr upload"));
    if (ok) {
        const size_t total = (size_t)(N / 16) * nbg * 64;
        const unsigned blocks = (unsigned)((total + 255) / 256);
        repack_kernel<<<blocks, 256>>>(draw, h->W, N, nblk, nbg, bits, raw_signed ? 1 : 0);
        ok = hip_ok(hipGetLastError(), "repack launch") &&
             hip_ok(hipDeviceSynchronize(), "repack");
    }
    if (draw) (void)hipFree(draw);
    if (!ok) {
        if (h->W) (void)hipFree(h->W);
        if (h->S) (void)hipFree(h->S);
        if (h->Z) (void)hipFree(h->Z);
        if (h->D) (void)hipFree(h->D);
        delete h;
        return nullptr;
    }
    h->dev_bytes = wbytes + sc_compact.size() * 4 + zp.size() + delta.size() * 4;
    return h;
}

template <int BITS, bool HP>
hipError_t launch_qmm_bits(const Handle* h, const QmmArgs& a, dim3 grid, hipStream_t st, bool dots) {
    const dim3 block(kWaves * 64);
#define QMM_LAUNCH(ZP, DL, DT) qmm_kernel<BITS, HP, ZP, DL, DT><<<grid, block, 0, st>>>(a)
    if (dots) {
        if (h->has_zp) {
            if (h->has_dl) QMM_LAUNCH(true, true, true);
            else QMM_LAUNCH(true, false, true);
        } else {
            if (h->has_dl) QMM_LAUNCH(false, true, true);
            else QMM_LAUNCH(false, false, true);
        }
    } else {
        if (h->has_zp) {
            if (h->has_dl) QMM_LAUNCH(true, true, false);
            else QMM_LAUNCH(true, false, false);
        } else {
            if (h->has_dl) QMM_LAUNCH(false, true, false);
            else QMM_LAUNCH(false, false, false);
        }
    }
#undef QMM_LAUNCH
    return hipGetLastError();
}

// Quantize + block dots + epilogue for M rows on `st`.  Exactly one of
// dC / dCs is non-null.
int run(Handle* h, const float* dA, int M, float* dC, int32_t* dCs, hipStream_t st) {
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
    Workspace& w = g_ws[dev];
    const size_t rb = (size_t)M * h->nblk;
    if (rb > (size_t)std::numeric_limits<int>::max() / 4) {
        set_err("M*K too large");
        return -2;
    }
    if (!ensure_blocks(w, rb)) return -4;
    const bool hp = g_hi_prec != 0;
    const unsigned qb = (unsigned)((rb + 255) / 256);
    if (hp) quantize_kernel<true><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, w.aq, w.sa, w.sq);
    else quantize_kernel<false><<<qb, 256, 0, st>>>(dA, M, h->K, h->nblk, w.aq, w.sa, w.sq);
    if (!hip_ok(hipGetLastError(), "quantize launch")) return -5;

    QmmArgs a{};
    a.W = h->W;
    a.S = h->S;
    a.Z = h->Z;
    a.D = h->D;
    a.Aq = reinterpret_cast<const uint2*>(w.aq);
    a.Sa = w.sa;
    a.Sq = w.sq;
    a.C = dC;
    a.Cs = dCs;
    a.M = M;
    a.N = h->N;
    a.nblk = h->nblk;
    a.nbg = h->nbg;
    a.sc_shift = h->sc_shift;
    a.ngrp = h->ngrp;
    const dim3 grid(h->N / 16, (M + kRowsPerWG - 1) / kRowsPerWG);
    const bool dots = dCs != nullptr;
    hipError_t e;
    if (h->bits == 8) e = hp ? launch_qmm_bits<8, true>(h, a, grid, st, dots)
                             : launch_qmm_bits<8, false>(h, a, grid, st, dots);
    else e = hp ? launch_qmm_bits<4, true>(h, a, grid, st, dots)
                : launch_qmm_bits<4, false>(h, a, grid, st, dots);
    if (!hip_ok(e, "matmul launch")) return -5;
    return 0;
}

int run_argmax(Handle* h, const float* dC, int M, int64_t* dIdx, hipStream_t st) {
    if (M == 0) return 0;
    int dev = 0;
    (void)hipGetDevice(&dev);
    Workspace& w = g_ws[dev];
    const int nparts = (h->N + kArgmaxChunk - 1) / kArgmaxChunk;
    if (!grow(&w.parts, &w.parts_cap, (size_t)M * nparts, "argmax workspace")) return -4;
    argmax_partial_kernel<<<dim3(nparts, M), 256, 0, st>>>(dC, h->N, w.parts);
    argmax_final_kernel<<<M, 256, 0, st>>>(w.parts, nparts, dIdx);
    return hip_ok(hipGetLastError(), "argmax launch") ? 0 : -5;
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
    if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(&qmm_kernel<8, true, false, false, false>)) !=
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
        return build_handle(reinterpret_cast<const uint8_t*>(b.data()), true, sc.data(), N, K, 8,
                            {}, delta);
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
    (void)hipSetDevice(cur);
    h->magic = 0;
    delete h;
}

int i4_matmul_dev(void* handle, const float* dA, int M, float* dC, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    return run(h, dA, M, dC, nullptr, static_cast<hipStream_t>(stream));
}

int i4_matmul_argmax_dev(void* handle, const float* dA, int M, float* dC, int64_t* dIdx, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    if (!dIdx) {
        set_err("null argmax output");
        return -2;
    }
    const int rc = run(h, dA, M, dC, nullptr, static_cast<hipStream_t>(stream));
    if (rc) return rc;
    return run_argmax(h, dC, M, dIdx, static_cast<hipStream_t>(stream));
}

int i4_block_dots_dev(void* handle, const float* dA, int M, int32_t* dCs, void* stream) {
    Handle* h = as_handle(handle);
    if (!h) return -1;
    return run(h, dA, M, nullptr, dCs, static_cast<hipStream_t>(stream));
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
    if (!grow(&w.hA, &w.hA_cap, na, "staging alloc") || !grow(&w.hC, &w.hC_cap, nc, "staging alloc"))
        return;
    if (!hip_ok(hipMemcpyAsync(w.hA, A, na * 4, hipMemcpyHostToDevice, w.stream), "upload A")) return;
    if (run(h, w.hA, M, w.hC, nullptr, w.stream) != 0) {
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
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < nblk; ++j)
                for (int oct = 0; oct < 4; ++oct) {
                    const int JG = bits == 8 ? 2 : 4;
                    const int t = n / 16, lane = oct * 16 + (n % 16), cg = j / JG, jb = j % JG;
                    const uint4 v = W[((size_t)t * h->nbg + cg) * 64 + lane];
                    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
                    if (bits == 8) {
                        uint8_t* dst = qw + ((size_t)n * nblk + j) * 32 + oct * 8;
                        const uint64_t x = (uint64_t)words[2 * jb + 1] << 32 | words[2 * jb];
                        for (int p = 0; p < 8; ++p) dst[kPerm8[p]] = (uint8_t)((x >> (8 * p)) ^ 0x80u);
                    } else {
                        uint8_t* dst = qw + ((size_t)n * nblk + j) * 16 + oct * 4;
                        for (int p = 0; p < 4; ++p) dst[p] = (uint8_t)(words[jb] >> (8 * p));
                    }
                }
    }
    if (scales) {
        std::vector<float> S((size_t)N * h->ngrp);
        if (!hip_ok(hipMemcpy(S.data(), h->S, S.size() * 4, hipMemcpyDeviceToHost), "download")) return -5;
        for (int n = 0; n < N; ++n)
            for (int j = 0; j < nblk; ++j)
                scales[(size_t)n * nblk + j] = S[(size_t)n * h->ngrp + (h->sc_shift == 31 ? 0 : j >> h->sc_shift)];
    }
    if (zp) {
        if (h->Z) {
            if (!hip_ok(hipMemcpy(zp, h->Z, blocks, hipMemcpyDeviceToHost), "download")) return -5;
        } else {
            std::memset(zp, bits == 8 ? 128 : 8, blocks);
        }
    }
    if (corr_delta) {
        if (h->D) {
            if (!hip_ok(hipMemcpy(corr_delta, h->D, blocks * 4, hipMemcpyDeviceToHost), "download")) return -5;
        } else {
            std::memset(corr_delta, 0, blocks * 4);
        }
    }
    return 0;
}

}  // extern "C"

// dec8_kernel.h -- the decode GEMV in row groups of eight: one workgroup per
// (tile range, eight rows), so every weight chunk crosses from L2 to a CU
// once per eight rows.  Instantiated per (bits, activation mode) by
// dec_w{4,8}_{hp,lp}.hip.
#pragma once

#include "qmm_common.h"

namespace bq {

// Waves 0..13 produce, waves 14 and 15 fold (one activation row of each
// output lane's pair each).  A tile's K range is cut into phases of 14
// chunks; producer w takes chunk 14p + w of phase p.
//
// MFMA A operand (v_mfma_i32_16x16x32_i8): row 2m + s is record part s of
// activation row m (the h and l bytes of the two-pass mode; the INT8 values
// and zeros with INT8 activations), so output lane (col, grp) holds the
// part-0 and part-1 dots of rows 2 grp and 2 grp + 1.  The records come
// through the producer's register ring from a buffer the stand-alone
// quantizer writes in that operand order ([chunk][JG / 2][64 lanes][16 B]),
// not through LDS: eight rows of K = 12288 are 192 KB.  The bias term
// 128 * sum(b) of the two-pass product, which the four-row kernel takes from
// two constant A rows, comes from a second MFMA per block of a constant A
// operand with the same B operand.
// kP8, kRows8, dec8_pitch, dec8_lds and kRecCopy are in qmm_common.h (the host
// plans launches with them).

// One weight chunk of a producer with its activation records (JG blocks of
// 8 bytes per lane) and per-column metadata: one scale, or for EXTRA
// handles (explicit zero points, legacy corr, scale groups smaller than a
// chunk) the chunk's per-block scales, corr deltas and INT4 zero points.
template <int JG, bool EXTRA>
struct Unit8 {
    uint4 w;
    uint4 a[JG / 2];
    float sc[EXTRA ? JG : 1];
    int dl[EXTRA ? JG : 1];
    uint32_t zp;
    int c;  // chunk to compute; nbg or more: none (past the end)
};

// Leading arguments in SGPRs at wave launch (kernarg preload), as in
// dec_kernel.  misc = sc_shift | RG << 8 | xcd << 12 | phases per tile << 16
// (RG row groups of eight rows; xcd: the RG workgroups of a tile range share
// an XCD).  pM is all rows of the call.  Tiles: the first rem_t tile ranges
// own base_t + 1, the rest base_t.
// LREC: the workgroup copies its row group's records into LDS once and the
// producers read them there, instead of from L2 for every tile (a
// workgroup with several tiles otherwise streams the records once per tile,
// as many bytes as the INT8 weights).
template <int BITS, bool HP, bool EXTRA, int FUSE, bool LREC>
__global__ __launch_bounds__(kDecWaves * 64) void dec8_kernel(const uint4* pW, const float* pS, const uint4* pR,
                                                              int pbase_t, int pnblk, int pM, int pnbg, int prem_t,
                                                              int pngrp, int misc, GemvArgs args) {
    constexpr int JG = BITS == 8 ? 2 : 4;
    constexpr int NA = JG / 2;
    constexpr int PP = dec8_pitch(JG);
    constexpr int R = kDecRing;
    // FUSE (as in dec_kernel): plain, the gate/up pair (each tile's gate
    // then up projection, C = silu(gate) * up), or several projections of
    // the activation (tiles concatenated over the segment table).
    constexpr bool PAIR = FUSE == kFusePair, MULTI = FUSE == kFuseMulti;
    // STREAM: the plain kernel with non-temporal weight loads (the host takes
    // it where each tile is read by at most two row groups: more share the
    // weights through L2, which non-temporal fills serve worse).
    constexpr bool STREAM = FUSE == kFuseStream;
    static_assert(FUSE == kFusePlain || PAIR || MULTI || STREAM, "no norm in this kernel's prologue");
    typedef float fvec __attribute__((ext_vector_type(JG)));
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = pnblk, nbg = pnbg;
    const int nblk4 = (nblk + 3) / 4 * 4;
    const int sc_shift = misc & 31, npw = misc >> 16;
    const int RG = (misc >> 8) & 15;

    // Row group rg (rows 8 rg .. 8 rg + 7) of tile range g.  Workgroups are
    // dealt to the 8 XCDs in turn; with xcd set the RG row groups of a tile
    // range are blocks 8 (RG (g / 8) + rg) + g % 8, on one XCD, so the later
    // reads of each weight chunk hit its L2.
    int g, rg;
    if (RG == 1) {
        g = blockIdx.x;
        rg = 0;
    } else if ((misc >> 12) & 1) {
        const int b = blockIdx.x, q = b >> 3;
        g = (q / RG) * 8 + (b & 7);
        rg = q % RG;
    } else {
        g = blockIdx.x / RG;
        rg = blockIdx.x % RG;
    }
    const int m0 = kRows8 * rg;
    const int M = min(kRows8, pM - m0);  // rows of this workgroup
    pR += (size_t)rg * nbg * (JG / 2) * 64;

    // Block scales and sums of q first (at most two uint4 per thread per
    // array: 8 * nblk4 <= 8192).
    const int nmeta = M * nblk4 / 4;
    const uint4* gsa = reinterpret_cast<const uint4*>(args.Sa + (size_t)m0 * nblk4);
    const uint4* gsq = reinterpret_cast<const uint4*>(args.Sq + (size_t)m0 * nblk4);
    const int mi0 = min(tid, nmeta - 1), mi1 = min(tid + 1024, nmeta - 1);
    const bool two_meta = nmeta > 1024;
    uint4 ma0 = gsa[mi0], ma1 = ma0, mq0 = make_uint4(0u, 0u, 0u, 0u), mq1 = mq0;
    if (two_meta) ma1 = gsa[mi1];
    if (BITS == 4) {
        mq0 = gsq[mi0];
        if (two_meta) mq1 = gsq[mi1];
    }
    // LREC: the records (nbg * NA * 64 uint4, at most kRecCopy = 8 per
    // thread), all loads in flight before any store, in named registers (an
    // array assigned under these branches was placed in scratch).  Each
    // group of 1024 is taken or skipped by the whole workgroup; threads past
    // the end of a group re-read its last record.
    const int nrec = nbg * NA * 64;
    static_assert(kRecCopy == 8, "the copy spells out eight groups");
    uint4 rc0, rc1, rc2, rc3, rc4, rc5, rc6, rc7;
    auto ldr = [&](int k, uint4& v) {
        if (1024 * k < nrec) v = pR[min(tid + 1024 * k, nrec - 1)];
    };
    if constexpr (LREC) {
        ldr(0, rc0);
        ldr(1, rc1);
        ldr(2, rc2);
        ldr(3, rc3);
        ldr(4, rc4);
        ldr(5, rc5);
        ldr(6, rc6);
        ldr(7, rc7);
    }
    __builtin_amdgcn_sched_barrier(0);

    const int t_begin = g * pbase_t + min(g, prem_t);
    const int nT = pbase_t + (g < prem_t ? 1 : 0);
    const int U = nT * npw * (PAIR ? 2 : 1);  // phases of this workgroup

    const Dec8Lds lay = dec8_lds(nblk, JG);
    float* sa_l = reinterpret_cast<float*>(smem + lay.sa);
    int* sq_l = reinterpret_cast<int*>(smem + lay.sq);
    float* fbuf = reinterpret_cast<float*>(smem + lay.fbuf);  // [2][2][64][PP]
    uint4* rec_l = reinterpret_cast<uint4*>(smem + lay.recs);   // LREC
    const int col = lane & 15, grp = lane >> 4;

    // Rows land at the padded pitch; sums of q premultiplied by -8 (the
    // default zero point) or by -1 (EXTRA: times each block's zero point in
    // the epilogue).  Threads past the end rewrite the last element.
    auto store_meta = [&]() {
        const int pad = (lay.sa_pitch - nblk4) >> 2;
        auto put = [&](int i, const uint4& va, const uint4& vq) {
            const int e = 4 * i;
            int m = 0;
#pragma unroll
            for (int r = 1; r < kRows8; ++r) m += e >= r * nblk4;
            const int d = i + m * pad;
            reinterpret_cast<uint4*>(sa_l)[d] = va;
            if (BITS == 4) {
                const uint32_t f = EXTRA ? 0xFFFFFFFFu : 0xFFFFFFF8u;  // -1 or -8
                reinterpret_cast<uint4*>(sq_l)[d] = make_uint4(f * vq.x, f * vq.y, f * vq.z, f * vq.w);
            }
        };
        put(mi0, ma0, mq0);
        if (two_meta) put(mi1, ma1, mq1);
        if constexpr (LREC) {
            auto str = [&](int k, const uint4& v) {
                if (1024 * k < nrec && tid + 1024 * k < nrec) rec_l[tid + 1024 * k] = v;
            };
            str(0, rc0);
            str(1, rc1);
            str(2, rc2);
            str(3, rc3);
            str(4, rc4);
            str(5, rc5);
            str(6, rc6);
            str(7, rc7);
        }
    };

    // Load cursor (as in dec_kernel): chunk ld_c of local tile ld_t, ld_rem
    // units before the tile ends; past the end ld_c is out of range and the
    // loads re-read the last tile.  A load with no work in a tile's short
    // last phase reads the chunk this producer loads in the next tile (L2
    // warm-up), or on the last tile the tile's last chunk.
    // PAIR: ld_sel selects the up projection of the current tile.  MULTI:
    // the weights and scales of segment ld_k are at lw and ls, and the
    // cursor moves to the next segment's arrays when a tile crosses into it
    // (the idle loads never leave a tile in either mode).
    int ld_c = wave, ld_rem = npw, ld_t = 0, ld_sel = 0;
    int ld_k = 0, t_off = 0;
    if (MULTI) {
        ld_k = (t_begin >= args.seg_end[0]) + (t_begin >= args.seg_end[1]) + (t_begin >= args.seg_end[2]);
        t_off = ld_k ? args.seg_end[ld_k - 1] : 0;
    }
    const uint4* lw = MULTI ? args.segW[ld_k] : pW;
    const float* ls = MULTI ? args.segS[ld_k] : pS;
    uint32_t ld_w = (uint32_t)(t_begin - t_off) * nbg * 64;
    uint32_t ld_s = (uint32_t)(t_begin - t_off) * pngrp * 16;
    uint32_t ld_m = (uint32_t)t_begin * nbg * 16;  // per-block metadata (EXTRA)
    const int pf_c = nbg + kP8 + wave;
    const bool pf = !PAIR && !MULTI && npw >= 2 && wave + kP8 < nbg;
    int ld_idle = (pf && nT > 1) ? pf_c : nbg - 1;
    auto load_unit = [&](Unit8<JG, EXTRA>& p) {
        const int c = min(ld_c, nbg - 1);
        const int cw = ld_c < nbg ? ld_c : ld_idle;
        uint32_t wi = ld_w + cw * 64 + lane;
        uint32_t si = ld_s + (uint32_t)((c * JG) >> sc_shift) * 16 + col;
        uint32_t ri = (uint32_t)c * (NA * 64) + lane;
        uint32_t mi = ld_m + c * 16 + col;
        asm("" : "+v"(wi), "+v"(si), "+v"(ri), "+v"(mi));
        const bool up = PAIR && ld_sel;
        if constexpr (STREAM) {
            typedef unsigned int u4v __attribute__((ext_vector_type(4)));
            const u4v t = __builtin_nontemporal_load(reinterpret_cast<const u4v*>(lw + wi));
            p.w = make_uint4(t.x, t.y, t.z, t.w);
        } else {
            p.w = (up ? args.W2 : lw)[wi];
        }
        if constexpr (!LREC) {
#pragma unroll
            for (int h = 0; h < NA; ++h) p.a[h] = pR[ri + 64 * h];
        }
        if constexpr (EXTRA) {
            typedef int ivec __attribute__((ext_vector_type(JG)));
            const fvec sv = *reinterpret_cast<const fvec*>((up ? args.S2 : args.S) + (size_t)mi * JG);
            const ivec dv = *reinterpret_cast<const ivec*>((up ? args.D2 : args.D) + (size_t)mi * JG);
#pragma unroll
            for (int jb = 0; jb < JG; ++jb) {
                p.sc[jb] = sv[jb];
                p.dl[jb] = dv[jb];
            }
            if (JG == 4) p.zp = *reinterpret_cast<const uint32_t*>((up ? args.Z2 : args.Z) + (size_t)mi * 4);
        } else {
            p.sc[0] = (up ? args.S2 : ls)[si];
        }
        p.c = ld_c;
        ld_c += kP8;
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
                    ld_s += pngrp * 16;
                    ld_m += nbg * 16;
                    if (MULTI && t_begin + ld_t == args.seg_end[ld_k]) {
                        ++ld_k;
                        lw = args.segW[ld_k];
                        ls = args.segS[ld_k];
                        ld_w = 0;
                        ld_s = 0;
                    }
                    if (ld_t + 1 == nT) ld_idle = nbg - 1;
                } else {
                    ld_c = 1 << 24;
                }
            }
        }
    };

    if (wave >= kP8) {
        // ================= chain waves: wave 14 folds row 2 grp, wave 15
        // row 2 grp + 1 of each lane's pair.  The fold is one dependent FMA
        // chain per output and paces the phases: first pick of the SIMD's
        // issue slots.
        __builtin_amdgcn_s_setprio(3);
        store_meta();
        lds_barrier();
        const int r = wave - kP8, row = 2 * grp + r;
        const float* sa_row = sa_l + row * lay.sa_pitch;
        const bool tail_pad = nblk != nbg * JG;  // the last chunk has padding blocks
        float acc = 0.0f, gate = 0.0f;
        unsigned long long best = 0;
        int pr_t = 0, pr_p = 0, pr_sel = 0, pr_k = 0;
        for (int u = 0; u < U; ++u) {
            lds_barrier();
            const float* fp = fbuf + (((u & 1) * 2 + r) * 64 + lane) * PP;
            const int c0 = kP8 * pr_p;
            const float* sp = sa_row + c0 * JG;
            if (c0 + kP8 < nbg || (c0 + kP8 == nbg && !tail_pad)) {
                // Full phase: all reads, then the FMAs in block order.
                fvec fv[kP8], sv[kP8];
#pragma unroll
                for (int i = 0; i < kP8; ++i) {
                    fv[i] = *reinterpret_cast<const fvec*>(fp + i * JG);
                    sv[i] = *reinterpret_cast<const fvec*>(sp + i * JG);
                }
#pragma unroll
                for (int i = 0; i < kP8; ++i) {
#pragma unroll
                    for (int jb = 0; jb < JG; ++jb) acc = __builtin_fmaf(sv[i][jb], fv[i][jb], acc);
                }
            } else {
                // The tile's last phase: whole chunks two at a time, then
                // the blocks of a padded last chunk.
                const int nb = nblk - c0 * JG, nwc = nb / JG;
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
                    // times the up projection (qwen35_decoder.cpp:408): the
                    // same expression as dec_kernel's.
                    const float v = PAIR ? silu_mul(gate, acc) : acc;
                    const int gt = t_begin + pr_t;
                    if (MULTI) {
                        while (gt >= args.seg_end[pr_k]) ++pr_k;
                        if (row < M) {
                            const int t0k = pr_k ? args.seg_end[pr_k - 1] : 0;
                            args.segC[pr_k][(size_t)(m0 + row) * args.segN[pr_k] + (gt - t0k) * 16 + col] = v;
                        }
                    } else {
                        const int n = gt * 16 + col;
                        if (row < M) args.C[(size_t)(m0 + row) * args.N + n] = v;
                        if (!PAIR && args.idx) {
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
        if (!PAIR && !MULTI && args.idx) {
            // Argmax as in dec_kernel: row maximum over the row's 16 lanes,
            // merged into the device's keys with device-scope atomic max;
            // after its atomics each chain wave takes a ticket, and the wave
            // holding the last of the grid's 2 * gridDim.x tickets swaps the
            // keys back to zero (re-arming them) and writes the indices.
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) {
                const unsigned long long o = __shfl_xor(best, sh, 16);
                best = o > best ? o : best;
            }
            if (col == 0 && row < M) (void)atomicMax(args.key + m0 + row, best);
            __builtin_amdgcn_s_waitcnt(0);
            unsigned int t = 0;
            if (lane == 0) t = atomicAdd(args.ticket, 1u);
            t = __shfl(t, 0);
            if (t == 2 * gridDim.x - 1 && lane < pM) {
                const unsigned long long k = atomicExch(args.key + lane, 0ull);
                args.idx[lane] = (int64_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
                if (lane == 0) atomicExch(args.ticket, 0u);
            }
        }
        return;
    }

    // ================= producers (waves 0..13)
    Unit8<JG, EXTRA> ring[R];
#pragma unroll
    for (int d = 0; d < R; ++d) load_unit(ring[d]);
    __builtin_amdgcn_sched_barrier(0);
    store_meta();
    lds_barrier();

    const int* sq0 = sq_l + (2 * grp) * lay.sa_pitch;
    const int* sq1 = sq0 + lay.sa_pitch;
    float* const fout = fbuf + lane * PP + wave * JG;
    // Constant A operand of the bias MFMA: rows 4 g + 1 and 4 g + 3 (odd
    // lanes' rows) all 64, the others zero.
    const long k64 = (lane & 1) ? 0x4040404040404040l : 0l;

    auto consume = [&](const Unit8<JG, EXTRA>& cur, int buf) {
        const int c = cur.c;
        if (c >= nbg) return;
        uint4 av[NA];
#pragma unroll
        for (int h = 0; h < NA; ++h) av[h] = LREC ? rec_l[(c * NA + h) * 64 + lane] : cur.a[h];
        // -8 * sum(q) (or -sum(q) with EXTRA) of rows 2 grp and 2 grp + 1
        // (INT4).
        int4 z0 = make_int4(0, 0, 0, 0), z1 = z0;
        if (BITS == 4) {
            z0 = *reinterpret_cast<const int4*>(sq0 + c * 4);
            z1 = *reinterpret_cast<const int4*>(sq1 + c * 4);
        }
        fvec f0, f1;
#pragma unroll
        for (int jb = 0; jb < JG; ++jb) {
            // Blocks past nblk (last chunk) read padding; the chain never
            // folds them.
            const uint64_t bop = unpack_b(cur.w, jb, BITS);
            const uint4& a2 = av[jb >> 1];
            const uint64_t aop = (jb & 1) ? ((uint64_t)a2.w << 32 | a2.z) : ((uint64_t)a2.y << 32 | a2.x);
            int e0 = 0, e1 = 0;
            if (BITS == 4) {
                e0 = jb == 0 ? z0.x : jb == 1 ? z0.y : jb == 2 ? z0.z : z0.w;
                e1 = jb == 0 ? z1.x : jb == 1 ? z1.y : jb == 2 ? z1.z : z1.w;
                if (EXTRA) {
                    const int zp = (int)(int8_t)(cur.zp >> (8 * jb));  // the block's zero point
                    e0 *= zp;
                    e1 *= zp;
                }
            }
            if (EXTRA) {
                // The legacy corr delta, in units of the part-1 (low byte)
                // dot: 256 of them per unit of the two-pass product.
                const int d = (HP ? 256 : 1) * cur.dl[EXTRA ? jb : 0];
                e0 += d;
                e1 += d;
            }
            const v4i dd = mfma16(aop, bop);
            int cs0 = dd[0] + e0, cs1 = dd[2] + e1;
            if constexpr (HP) {
                // 128 * sum(b) from a 16x16x32 MFMA of the constant A
                // operand (rows 4 g + 1 and 4 g + 3 all 64) with the same B
                // operand: results 1 and 3 of every output lane are each
                // 64 * sum(b) of its column.  Both MFMAs take a zero
                // accumulator input and the sums are VALU adds (an MFMA
                // result fed straight into the next MFMA's accumulator input
                // was allocated with partial register overlaps).
                const v4i bs = __builtin_amdgcn_mfma_i32_16x16x32_i8(k64, (long)bop, v4i{0, 0, 0, 0}, 0, 0, 0);
                const int s128 = bs[1] + bs[3];
                cs0 = dd[0] * 256 + dd[1] + (s128 + e0);
                cs1 = dd[2] * 256 + dd[3] + (s128 + e1);
            }
            const float sc = cur.sc[EXTRA ? jb : 0];
            f0[jb] = (float)cs0 * sc;
            f1[jb] = (float)cs1 * sc;
        }
        *reinterpret_cast<fvec*>(fout + (buf * 2) * 64 * PP) = f0;
        *reinterpret_cast<fvec*>(fout + (buf * 2 + 1) * 64 * PP) = f1;
    };

    for (int u0 = 0; u0 < U; u0 += R) {
#pragma unroll
        for (int d = 0; d < R; ++d) {
            const bool live = u0 + d < U;  // uniform over the workgroup
            consume(ring[d], (u0 + d) & 1);
            load_unit(ring[d]);
            __builtin_amdgcn_sched_barrier(0);
            if (live) lds_barrier();
        }
    }
}

template <int BITS, bool HP, bool EXTRA, int FUSE, bool LREC>
hipError_t launch_dec8_f(bool* attr_set, const GemvArgs& a, const uint4* rec, int grid, int lds, hipStream_t st) {
    auto kern = dec8_kernel<BITS, HP, EXTRA, FUSE, LREC>;
    bool& set = attr_set[(FUSE == kFuseStream ? 3 : FUSE) + (EXTRA ? 4 : 0) + (LREC ? 8 : 0)];
    if (!set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
        if (e != hipSuccess) return e;
        set = true;
    }
    const int npw = (a.nbg + kP8 - 1) / kP8;
    const int misc = a.sc_shift | a.RG << 8 | a.pair_xcd << 12 | npw << 16;
    const int base_t = a.ntiles / a.NG, rem_t = a.ntiles - base_t * a.NG;
    kern<<<grid, kDecWaves * 64, lds, st>>>(a.W, a.S, rec, base_t, a.nblk, a.M, a.nbg, rem_t, a.ngrp, misc, a);
    return hipGetLastError();
}

// attr_set: this device's flags for the (bits, mode) pair, one per (FUSE
// mode, per-block metadata, records in LDS) variant (16 a pair).  Handles with per-block
// metadata take the plain and paired calls (the multi-projection launch
// sends them one by one).
template <int BITS, bool HP, bool LREC>
hipError_t launch_dec8_l(bool* attr_set, const GemvArgs& a, const uint4* rec, int grid, int lds, int fuse, bool extra,
                         hipStream_t st) {
    if (extra) {
        if (fuse == kFusePair) return launch_dec8_f<BITS, HP, true, kFusePair, LREC>(attr_set, a, rec, grid, lds, st);
        if (fuse == kFuseStream) return launch_dec8_f<BITS, HP, true, kFuseStream, LREC>(attr_set, a, rec, grid, lds, st);
        if (fuse != kFusePlain) return hipErrorInvalidValue;
        return launch_dec8_f<BITS, HP, true, kFusePlain, LREC>(attr_set, a, rec, grid, lds, st);
    }
    if (fuse == kFusePair) return launch_dec8_f<BITS, HP, false, kFusePair, LREC>(attr_set, a, rec, grid, lds, st);
    if (fuse == kFuseMulti) return launch_dec8_f<BITS, HP, false, kFuseMulti, LREC>(attr_set, a, rec, grid, lds, st);
    if (fuse == kFuseStream) return launch_dec8_f<BITS, HP, false, kFuseStream, LREC>(attr_set, a, rec, grid, lds, st);
    if (fuse != kFusePlain) return hipErrorInvalidValue;
    return launch_dec8_f<BITS, HP, false, kFusePlain, LREC>(attr_set, a, rec, grid, lds, st);
}

template <int BITS, bool HP>
hipError_t launch_dec8(bool* attr_set, const GemvArgs& a, const uint4* rec, int grid, int lds, int fuse, bool extra,
                       bool lrec, hipStream_t st) {
    return lrec ? launch_dec8_l<BITS, HP, true>(attr_set, a, rec, grid, lds, fuse, extra, st)
                : launch_dec8_l<BITS, HP, false>(attr_set, a, rec, grid, lds, fuse, extra, st);
}

}  // namespace bq

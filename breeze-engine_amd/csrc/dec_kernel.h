// dec_kernel.h -- the decode GEMV kernel (up to 32 rows) and its launcher,
// instantiated per (bits, activation mode) by dec_w{4,8}_{hp,lp}.hip.
#pragma once

#include "qmm_common.h"

namespace bq {

// The leading scalar arguments are what the first activation and weight
// loads need.  They are preloaded into SGPRs at wave launch (kernarg
// preload, 14 SGPRs), so those loads do not wait for a kernarg fetch; the
// rest of the arguments come from the struct as the code reaches them.
// Tiles per workgroup group: the first rem_t groups own base_t + 1 tiles, the
// rest base_t (ntiles = base_t * NG + rem_t).  misc = sc_shift | log2(4 / RS)
// << 5 | RG << 8 | xcd << 12 | phases per tile << 16 (RG row groups of RS
// rows, RS 4, 2 or 1, RG up to 8; xcd: the RG workgroups of one tile range
// share an XCD).  PAIR: gate and up projections
// in one launch; each output tile is the gate tile then the up tile of the
// same columns, and C = silu(gate) * up.
//
// SPLIT (split-K, one row group): workgroup b takes piece b % S of tile
// b / S, where S = prem_t and the S pieces are balanced ranges of the
// tile's phases.  It quantizes only its piece's blocks, stores each block's
// value f = (float)cs * scale and the activation scales to the tile's
// region of sf instead of folding them, and takes a ticket.  The last of
// the tile's S workgroups folds every block in order, acc = fma(sa, f,
// acc) as in the unsplit fold (quantized_matmul.cpp:311-315), so the
// output is the same bits, and re-arms the ticket.  No workgroup waits for
// another.

template <int BITS, bool HP, bool FUSED, bool EXTRA, int R, int FUSE, bool P64>
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
    a.RS = 4 >> ((misc >> 5) & 3);
    a.RG = (misc >> 8) & 15;
    a.pair_xcd = (misc >> 12) & 1;
    constexpr bool PAIR = FUSE == kFusePair || FUSE == kFusePairFlow || FUSE == kFusePairFlowStream;
    constexpr bool NORM = FUSE == kFuseNormMulti;
    constexpr bool MULTI = FUSE == kFuseMulti || NORM;
    constexpr bool SPLIT = FUSE == kFuseSplit;
    // Weight chunks are read once per call: with STREAM the loads carry the
    // non-temporal hint, which streams faster where a workgroup reads many
    // tiles (the host decides; the idle loads' L2 re-reads then miss more,
    // which costs where it has few).
    constexpr bool STREAM = FUSE == kFuseStream || FUSE == kFuseFlowStream || FUSE == kFusePairFlowStream;
    // FLOW: phases run across tile boundaries (the host takes it where
    // workgroups hold several tiles of at least 15 whole chunks); with PAIR
    // the stream alternates a column tile's gate and up chunks.
    constexpr bool FLOW = FUSE == kFuseFlow || FUSE == kFuseFlowStream || FUSE == kFusePairFlow ||
                          FUSE == kFusePairFlowStream;
    static_assert(!SPLIT || FUSED, "split-K quantizes its pieces in the prologue");
    constexpr int JG = BITS == 8 ? 2 : 4;
    constexpr int PP = dec_pitch(JG);
    typedef float fvec __attribute__((ext_vector_type(JG)));
    typedef int ivec __attribute__((ext_vector_type(JG)));
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    const int npw = misc >> 16;  // phases per tile: ceil(nbg / 15)
    const int nsplit = SPLIT ? prem_t : 1;
    int g, rg, piece = 0;
    if (SPLIT) {
        g = blockIdx.x / nsplit;
        piece = blockIdx.x - g * nsplit;
        rg = 0;
    } else if (a.RG == 1) {
        g = blockIdx.x;
        rg = 0;
    } else if (a.pair_xcd) {
        // Workgroups are dealt to the 8 XCDs in turn: the RG row groups of
        // tile range g are blocks 8 (RG (g / 8) + rg) + g % 8, one XCD.
        const int b = blockIdx.x, q = b >> 3;
        g = (q / a.RG) * 8 + (b & 7);
        rg = q % a.RG;
    } else {
        g = blockIdx.x / a.RG;
        rg = blockIdx.x % a.RG;
    }
    const int m0 = rg * a.RS;
    const int Mr = min(a.RS, a.M - m0);
    // Phases [pa, pb) of each tile; with SPLIT the piece's blocks
    // [qb0, qb0 + nbr) of each row are the ones quantized, and LDS holds
    // them (records, scales, sums) from the piece's first block and chunk
    // coff on.
    const int pa = SPLIT ? piece * npw / nsplit : 0, pb = SPLIT ? (piece + 1) * npw / nsplit : npw;
    const int qb0 = SPLIT ? pa * kProducers * JG : 0;
    const int coff = SPLIT ? pa * kProducers : 0;
    const int nbr = SPLIT ? min(pb * kProducers * JG, pnblk) - qb0 : pnblk;

    // Activation loads, ahead of all other set-up in program order: at kernel
    // start the prologue's instructions are fetched cold, and timestamps put
    // the load ~1.4 us after wave start when it sat behind the set-up code.
    // K is a multiple of 32, so the rows m0.. of A are nb_rows contiguous
    // 32-float blocks, and the staged scale and sum rows (pitch nblk4) are
    // contiguous too: a block index is an offset, with no row/column split.
    const int nb_rows = Mr * nbr;
    // Lane q = tid & 3 of a quad holds k = 8q..8q+7 of its block: two uint4
    // per pass, every pass's loads in flight before the first is quantized.
    // The array is indexed only by constants after unrolling, so it stays in
    // registers.
    Oct av[kQuantPasses];
    Oct wn0, wn1;  // NORM (at most two passes): the norm weights of those elements
    uint4 r0, r1, r2, r3, r4, r5, rsa, rsq;  // named: an indexed array would live in scratch
    if (FUSED) {
        if (nb_rows > kQuantEarlyBlocks || wave < 8) {
            const float* arow = a.A + (size_t)m0 * a.K + 8 * (tid & 3);
            const bool all = nb_rows > kQuantEarlyBlocks;
            const int qb = all ? 256 : 128;  // blocks per pass
            const int npass = all ? (nb_rows + 255) >> 8 : 1;
            const bool two = npass > 1;
            auto ld = [&](int p, Oct& v) {
                int blk = min(p * qb + (tid >> 2), nb_rows - 1);
                if (SPLIT) {
                    // Row m's piece starts at block qb0 of that row.
                    const int m = (blk >= nbr) + (blk >= 2 * nbr) + (blk >= 3 * nbr);
                    blk += qb0 + m * (pnblk - nbr);
                }
                v.x = *reinterpret_cast<const uint4*>(arow + 32 * blk);
                v.y = *reinterpret_cast<const uint4*>(arow + 32 * blk + 4);
            };
#pragma unroll
            for (int p = 0; p < kQuantPasses; ++p)
                if (p < npass) ld(p, av[p]);
            if (NORM) {
                auto ldw = [&](int p, Oct& v) {
                    const int blk = min(p * qb + (tid >> 2), nb_rows - 1);
                    const int m = (blk >= a.nblk) + (blk >= 2 * a.nblk) + (blk >= 3 * a.nblk);
                    const float* wrow = a.normW + 32 * (blk - m * a.nblk) + 8 * (tid & 3);
                    v.x = *reinterpret_cast<const uint4*>(wrow);
                    v.y = *reinterpret_cast<const uint4*>(wrow + 4);
                };
                ldw(0, wn0);
                if (two) ldw(1, wn1);
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

    const int base_t = pbase_t, rem_t = SPLIT ? 0 : prem_t;
    const int t_begin = g * base_t + min(g, rem_t);
    const int nT = base_t + (g < rem_t ? 1 : 0);
    const int nbg = a.nbg;
    const int U = SPLIT  ? pb - pa
                  : FLOW ? (nT * nbg * (PAIR ? 2 : 1) + kProducers - 1) / kProducers
                         : nT * npw * (PAIR ? 2 : 1);  // phases of this workgroup

    const DecLds lay = dec_lds(min(a.M, a.RS), SPLIT ? split_piece_blocks(npw, nsplit, a.nbg, JG) : a.nblk, JG, P64);
    uint8_t* recs = smem + lay.recs;
    float* sa_l = reinterpret_cast<float*>(smem + lay.sa);
    int* sq_l = reinterpret_cast<int*>(smem + lay.sq);
    float* fbuf = reinterpret_cast<float*>(smem + lay.fbuf);  // [2][64][PP]

    const int col = lane & 15, grp = lane >> 4;
    const int me = min(grp, Mr - 1);

    // SPLIT: the folding workgroup copies its tile's region of sf to LDS
    // (pitch split_pitch) with device-scope loads, which see every piece's
    // device-scope stores; sixteen in flight per thread (128 KB a round).
    auto split_stage = [&]() {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(a.sf + (size_t)g * a.M * 17 * a.nblk4);
        const int q2 = a.nblk4 >> 1, n2 = a.M * 17 * q2, P = split_pitch(a.nblk4);
        float* st = reinterpret_cast<float*>(smem);
        constexpr int kIn = 16;
        for (int i0 = 0; i0 < n2; i0 += kIn * kDecWaves * 64) {
            uint64_t v[kIn];  // indexed by constants only: registers
            // Groups wholly past the region are skipped (a uniform branch);
            // the last group's extra threads re-read its last element.
#pragma unroll
            for (int k = 0; k < kIn; ++k)
                if (i0 + k * kDecWaves * 64 < n2)
                    v[k] = __hip_atomic_load(src + min(i0 + k * kDecWaves * 64 + tid, n2 - 1), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int k = 0; k < kIn; ++k) {
                const int i = i0 + k * kDecWaves * 64 + tid;
                if (i < n2) {
                    const int r = i / q2, q = i - r * q2;
                    *reinterpret_cast<uint64_t*>(st + r * P + 2 * q) = v[k];
                }
            }
        }
    };

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
    //
    // With several projections (MULTI) the weights and scales of segment
    // ld_k are at lw and ls; the cursor moves to the next segment's arrays
    // when a tile crosses into it, and the idle loads never leave a tile.
    int ld_c = wave + kProducers * pa, ld_rem = pb - pa, ld_t = 0, ld_sel = 0;  // ld_sel: up tile of a pair
    int ld_k = 0, t_off = 0;  // MULTI: segment of the next tile, and its first tile
    if (MULTI) {
        ld_k = (t_begin >= args.seg_end[0]) + (t_begin >= args.seg_end[1]) + (t_begin >= args.seg_end[2]);
        t_off = ld_k ? args.seg_end[ld_k - 1] : 0;
    }
    const uint4* lw = MULTI ? args.segW[ld_k] : a.W;
    const float* ls = MULTI ? args.segS[ld_k] : a.S;
    uint32_t ld_w = (uint32_t)(t_begin - t_off) * nbg * 64;
    uint32_t ld_s = (uint32_t)(t_begin - t_off) * a.ngrp * 16;
    uint32_t ld_m = (uint32_t)t_begin * nbg * 16;
    const int pf_c = nbg + kProducers + wave;
    const bool pf = !PAIR && !MULTI && !FLOW && npw >= 2 && wave + kProducers < nbg;
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
        if constexpr (STREAM) {
            typedef unsigned int u4v __attribute__((ext_vector_type(4)));
            const u4v t = __builtin_nontemporal_load(reinterpret_cast<const u4v*>((up ? a.W2 : lw) + wi));
            p.w = make_uint4(t.x, t.y, t.z, t.w);
        } else {
            p.w = (up ? a.W2 : lw)[wi];
        }
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
            p.sc[0] = (up ? a.S2 : ls)[si];
        }
        p.c = ld_c;
        ld_c += kProducers;
        if constexpr (FLOW) {
            // One stream of chunks over the tiles (nbg >= 15: one wrap at
            // most; a gate tile wraps into the same columns' up tile);
            // past the last tile the loads re-read its last chunk.
            if (ld_c >= nbg) {
                if (PAIR && ld_sel == 0) {
                    ld_sel = 1;
                    ld_c -= nbg;
                } else if (++ld_t < nT) {
                    if (PAIR) ld_sel = 0;
                    ld_c -= nbg;
                    ld_w += nbg * 64;
                    ld_s += a.ngrp * 16;
                    ld_m += nbg * 16;
                } else {
                    ld_c = 1 << 24;
                }
            }
        } else if (--ld_rem == 0) {
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

    // ---------------- prologue
    // The activation loads went out first (above); the first R weight units
    // follow, then the activations are quantized (or their records copied)
    // into LDS while the weights stream in.  The scheduling barriers keep
    // this issue order.
    auto store_acts = [&]() {
        if (FUSED) {
            const bool all = nb_rows > kQuantEarlyBlocks;
            const int qb = all ? 256 : 128;  // blocks per pass
            const int npass = all ? (nb_rows + 255) >> 8 : wave < 8 ? 1 : 0;  // 0 to kQuantPasses
            // NORM: the decoder's RMSNorm of each row first, hn = (x * inv) * w
            // with inv = 1 / sqrtf((float)(ss / K) + eps)
            // (kernel/qwen35_decoder.cpp:134-140), bit for bit.  The block
            // sums of squares (two runs of 4 terms in a lane, their sum, a
            // 4-lane DPP sum: the 8-lane sum of 4-term runs, pair by pair) go to
            // the idle phase buffer, every wave adds up each row's (a lane
            // run of at most 6, a 16-lane DPP sum, the 4 row sums by lane
            // swaps: at most 18 roundings a term) and norm_mean_from_bound_r
            // decides the mean; a row it does not decide takes the in-order
            // sum.  Any
            // summation order serves: the mean either comes from the bound,
            // which proves it equal to the reference's, or from the in-order
            // sum itself.
            float inv_r[NORM ? 4 : 1];
            if constexpr (NORM) {
                const double rK = 1.0 / (double)a.K;  // ahead of the loads' use: off the critical path
                double* nsq = reinterpret_cast<double*>(fbuf);
                auto sumsq = [&](int p, const Oct& v) {
                    const int blk = p * qb + (tid >> 2);
                    auto run4 = [](const uint4& u) {
                        const float x0 = __uint_as_float(u.x), x1 = __uint_as_float(u.y);
                        const float x2 = __uint_as_float(u.z), x3 = __uint_as_float(u.w);
                        double t = (double)x0 * (double)x0;
                        t += (double)x1 * (double)x1;
                        t += (double)x2 * (double)x2;
                        return t + (double)x3 * (double)x3;
                    };
                    double t = run4(v.x) + run4(v.y);
                    t += dpp_f64(t, 0xB1);  // lane ^ 1
                    t += dpp_f64(t, 0x4E);  // lane ^ 2
                    if ((tid & 3) == 0 && blk < nb_rows) nsq[blk] = t;
                };
                if (npass > 0) sumsq(0, av[0]);
                if (npass > 1) sumsq(1, av[1]);
                lds_barrier();
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    inv_r[r] = 0.0f;
                    if (r >= Mr || npass == 0) continue;
                    // A lane's run: at most 6 block sums (384 row-blocks),
                    // all read before the first add; the zeros past nblk
                    // add exactly.
                    double t[kNormRun];
#pragma unroll
                    for (int j = 0; j < kNormRun; ++j) {
                        const int i = lane + 64 * j;
                        t[j] = i < a.nblk ? nsq[r * a.nblk + i] : 0.0;
                    }
                    double v = t[0];
#pragma unroll
                    for (int j = 1; j < kNormRun; ++j) v += t[j];
                    v = sum_rows_f64(sum16_f64(v));
                    float mean;
                    if (a.norm_exact || a.nblk > 64 * kNormRun || !(v - v == 0.0) ||
                        !norm_mean_from_bound_r(v, a.K, rK, 0, &mean))
                        mean = (float)(norm_sumsq_inorder<8>(a.A + (size_t)(m0 + r) * a.K, a.K) / (double)a.K);
                    inv_r[r] = 1.0f / sqrtf(mean + a.norm_eps);
                }
            }
            auto qpass = [&](int p, const Oct& v, const Oct& w) {
                const int blk = p * qb + (tid >> 2), e = tid & 3;
                float s;
                int sum;
                uint2 ph, pl;
                float4 x0 = make_float4(__uint_as_float(v.x.x), __uint_as_float(v.x.y), __uint_as_float(v.x.z),
                                        __uint_as_float(v.x.w));
                float4 x1 = make_float4(__uint_as_float(v.y.x), __uint_as_float(v.y.y), __uint_as_float(v.y.z),
                                        __uint_as_float(v.y.w));
                if constexpr (NORM) {
                    const int m = (blk >= a.nblk) + (blk >= 2 * a.nblk) + (blk >= 3 * a.nblk);
                    const float inv = m == 0 ? inv_r[0] : m == 1 ? inv_r[1] : m == 2 ? inv_r[2] : inv_r[3];
                    auto nrm = [&](const float4& x, const uint4& w) {
                        return make_float4(x.x * inv * __uint_as_float(w.x), x.y * inv * __uint_as_float(w.y),
                                           x.z * inv * __uint_as_float(w.z), x.w * inv * __uint_as_float(w.w));
                    };
                    x0 = nrm(x0, w.x);
                    x1 = nrm(x1, w.y);
                    if (a.normOut && g == 0 && blk < nb_rows) {
                        float* o = a.normOut + (size_t)m0 * a.K + 32 * blk + 8 * e;
                        *reinterpret_cast<float4*>(o) = x0;
                        *reinterpret_cast<float4*>(o + 4) = x1;
                    }
                }
                quant4x8<HP>(x0, x1, s, ph, pl, sum);
                if (blk < nb_rows) {
                    const int m = (blk >= nbr) + (blk >= 2 * nbr) + (blk >= 3 * nbr), j = blk - m * nbr;
                    if (P64) {
                        // Lane e holds k-octet e: its slot is the zero
                        // half, then the octet.
                        uint4* sh = reinterpret_cast<uint4*>(recs + m * lay.rec_pitch + j * 128 + e * 16);
                        sh[0] = make_uint4(0u, 0u, ph.x, ph.y);
                        sh[4] = make_uint4(0u, 0u, pl.x, pl.y);  // l octets, 64 B further
                    } else {
                        // [chunk][h, l][k-octet][block of the chunk] of 8
                        // bytes: a lane's A operands for a chunk are 8 JG
                        // contiguous bytes.
                        uint8_t* rec = recs + m * lay.rec_pitch + (j / JG) * (JG * 64) + e * (JG * 8) + (j % JG) * 8;
                        *reinterpret_cast<uint2*>(rec) = ph;
                        *reinterpret_cast<uint2*>(rec + JG * 32) = pl;
                    }
                    if (e == 0) {
                        sa_l[m * lay.sa_pitch + j] = s;
                        sq_l[m * lay.sa_pitch + j] = (EXTRA ? -1 : -8) * sum;
                    }
                }
            };
#pragma unroll
            for (int p = 0; p < kQuantPasses; ++p)
                if (p < npass) qpass(p, av[p], p == 0 ? wn0 : wn1);
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
                    uint32_t* z = reinterpret_cast<uint32_t*>(recs + (tid >> 2) * lay.rec_pitch + nbr * 128);
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
        int pr_t = 0, pr_p = pa, pr_sel = 0, pr_k = 0;
        int tb = 0;  // FLOW: the stream's chunk index where tile pr_t starts
        // FLOW: a finished tile's outputs (and argmax keys).
        auto emit = [&](float v) {
            if (grp < Mr) {
                const int n = (t_begin + pr_t) * 16 + col;
                a.C[(size_t)(m0 + grp) * a.N + n] = v;
                if (a.idx) {
                    const unsigned long long k = argmax_key(v, n);
                    best = k > best ? k : best;
                }
            }
        };
        // FLOW: the stream's tile ends (with PAIR a gate tile's sum waits
        // for the same columns' up tile).
        auto tile_end = [&](float v) {
            if (PAIR && pr_sel == 0) {
                gate = v;
                pr_sel = 1;
            } else {
                emit(PAIR ? silu_mul(gate, v) : v);
                if (PAIR) pr_sel = 0;
                ++pr_t;
            }
            tb += nbg;
        };
        for (int u = 0; u < U; ++u) {
            lds_barrier();
            const float* fp = fbuf + ((u & 1) * 64 + lane) * PP;
            if constexpr (FLOW) {
                // Slot i holds chunk kProducers u + i of the stream: chunk
                // c0 + i of tile pr_t while that lasts.
                const int c0 = kProducers * u - tb, rem = nbg - c0;
                const float* sp = sa_row + c0 * JG;
                if (rem >= kProducers) {
                    // The phase lies in one tile, no padding: as the
                    // unsplit kernel's full phase.
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
                    if (rem == kProducers) {
                        tile_end(acc);
                        acc = 0.0f;
                    }
                } else {
                    // Tile pr_t ends at slot rem - 1 (no padding: the host
                    // takes FLOW only where nblk is whole chunks); the next
                    // tile's chunks 0.. follow from slot rem, or nothing
                    // after the last tile (those slots are folded into no
                    // output).  In two halves of slots (fewer registers
                    // live than the full phase), the tile's sum taken when
                    // slot rem begins.
                    float out = 0.0f;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        constexpr int kH = (kProducers + 1) / 2;
                        fvec fv[kH], sv[kH];
#pragma unroll
                        for (int k = 0; k < kH; ++k) {
                            const int i = h * kH + k;
                            if (i < kProducers) {
                                const int so = i < rem ? c0 + i : i - rem;
                                fv[k] = *reinterpret_cast<const fvec*>(fp + i * JG);
                                sv[k] = *reinterpret_cast<const fvec*>(sa_row + so * JG);
                            }
                        }
#pragma unroll
                        for (int k = 0; k < kH; ++k) {
                            const int i = h * kH + k;
                            if (i < kProducers) {
                                out = i == rem ? acc : out;
                                acc = i == rem ? 0.0f : acc;
#pragma unroll
                                for (int jb = 0; jb < JG; ++jb) acc = __builtin_fmaf(sv[k][jb], fv[k][jb], acc);
                            }
                        }
                    }
                    tile_end(out);
                }
                continue;
            }
            const int c0 = kProducers * pr_p;
            const float* sp = sa_row + (c0 - coff) * JG;
            if constexpr (SPLIT) {
                // The phase's block values (whole chunks: padding blocks of
                // a last chunk land inside the row's nblk4 and are never
                // folded), and the block scales from the column-0 lanes,
                // written through to device scope.
                if (grp < Mr) {
                    float* fo = a.sf + ((size_t)g * a.M + grp) * 17 * a.nblk4 + c0 * JG;
                    const int nch = min(kProducers, nbg - c0);
#pragma unroll
                    for (int i = 0; i < kProducers; ++i)
                        if (i < nch) store_agent<JG>(fo + col * a.nblk4 + i * JG, fp + i * JG);
                    if (col == 0) {
#pragma unroll
                        for (int i = 0; i < kProducers; ++i)
                            if (i < nch) store_agent<JG>(fo + 16 * a.nblk4 + i * JG, sp + i * JG);
                    }
                }
                ++pr_p;
                continue;
            }
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
                    const float v = PAIR ? silu_mul(gate, acc) : acc;
                    if (MULTI) {
                        // Tiles come in increasing order: step into the
                        // segment of this one.
                        const int gt = t_begin + pr_t;
                        while (gt >= args.seg_end[pr_k]) ++pr_k;
                        if (grp < Mr) {
                            const int t0k = pr_k ? args.seg_end[pr_k - 1] : 0;
                            args.segC[pr_k][(size_t)(m0 + grp) * args.segN[pr_k] + (gt - t0k) * 16 + col] = v;
                        }
                    } else if (grp < Mr) {
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
        if constexpr (SPLIT) {
            // The device-scope stores above complete before the ticket is
            // taken (the fence keeps the compiler from moving them past the
            // wait).  The holder of the last ticket folds the tile, reading
            // every piece's stores with device-scope loads.  No cache-wide
            // write-back or invalidation is needed: only these stores and
            // loads cross workgroups.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_waitcnt(0);
            unsigned int tk = 0;
            if (lane == 0) tk = atomicAdd(a.stick + g, 1u);
            tk = __shfl(tk, 0);
            const bool last = tk == (unsigned int)(nsplit - 1);
            int* flag = reinterpret_cast<int*>(smem + split_flag_off(a.M, a.nblk4, lay.total));
            if (lane == 0) *flag = last ? 1 : 0;
            lds_barrier();
            if (!last) return;
            split_stage();
            lds_barrier();
            if (grp < Mr) {
                // One dependent FMA per block; in whole batches of 16 the
                // next batch's reads are issued before the current batch's
                // FMAs (a read past the batches is clamped into the row:
                // its values are not used), then the rest block by block.
                const int P = split_pitch(a.nblk4);
                const float* st = reinterpret_cast<const float*>(smem);
                const float* fr = st + (grp * 17 + col) * P;
                const float* sr = st + (grp * 17 + 16) * P;
                float v = 0.0f;
                const int nfull = a.nblk & ~15;
                int b = 0;
                if (nfull > 0) {
                    float4 f0, f1, f2, f3, s0, s1, s2, s3;
                    auto rd = [&](int o, float4& x0, float4& x1, float4& x2, float4& x3, float4& y0, float4& y1,
                                  float4& y2, float4& y3) {
                        x0 = *reinterpret_cast<const float4*>(fr + o);
                        x1 = *reinterpret_cast<const float4*>(fr + o + 4);
                        x2 = *reinterpret_cast<const float4*>(fr + o + 8);
                        x3 = *reinterpret_cast<const float4*>(fr + o + 12);
                        y0 = *reinterpret_cast<const float4*>(sr + o);
                        y1 = *reinterpret_cast<const float4*>(sr + o + 4);
                        y2 = *reinterpret_cast<const float4*>(sr + o + 8);
                        y3 = *reinterpret_cast<const float4*>(sr + o + 12);
                    };
                    auto fma4 = [&](const float4& x, const float4& y) {
                        v = __builtin_fmaf(y.x, x.x, v);
                        v = __builtin_fmaf(y.y, x.y, v);
                        v = __builtin_fmaf(y.z, x.z, v);
                        v = __builtin_fmaf(y.w, x.w, v);
                    };
                    float4 g0, g1, g2, g3, t0, t1, t2, t3;
                    rd(0, f0, f1, f2, f3, s0, s1, s2, s3);
                    // Two batches an iteration: each half reads the batch
                    // after next while the FMAs consume the one read before.
                    for (; b + 32 <= nfull; b += 32) {
                        rd(b + 16, g0, g1, g2, g3, t0, t1, t2, t3);
                        fma4(f0, s0);
                        fma4(f1, s1);
                        fma4(f2, s2);
                        fma4(f3, s3);
                        rd(min(b + 32, P - 16), f0, f1, f2, f3, s0, s1, s2, s3);
                        fma4(g0, t0);
                        fma4(g1, t1);
                        fma4(g2, t2);
                        fma4(g3, t3);
                        // Keep each half's reads ahead of its FMAs (the
                        // scheduler would move them next to their uses).
                        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                    }
                    if (b < nfull) {  // one batch left, already read
                        fma4(f0, s0);
                        fma4(f1, s1);
                        fma4(f2, s2);
                        fma4(f3, s3);
                        b += 16;
                    }
                }
                for (; b < a.nblk; ++b) v = __builtin_fmaf(sr[b], fr[b], v);
                a.C[(size_t)grp * a.N + g * 16 + col] = v;
            }
            if (lane == 0) (void)atomicExch(a.stick + g, 0u);
            return;
        }
        if (!PAIR && !MULTI && a.idx) {
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

    // Computes one unit into phase buffer buf.
    auto consume = [&](const Unit<JG, EXTRA>& cur, int buf) {
        const int c = cur.c;
        if (P64 && c < nbg) {
            const int abase = p_data ? p_data_base + (c - coff) * JG * 128 : p_const_base;
            int2 nsq2 = make_int2(0, 0);  // this lane's block in each pair
            if (BITS == 4) {
                const int* q = sq_l + o_row * lay.sa_pitch + (c - coff) * 4 + o_sel;
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
            const int abase = is_data ? data_base + (c - coff) * JG * 64 : const_base;
            // The chunk's JG A operands of this lane: 8 JG contiguous bytes.
            uint4 av4[JG / 2];
#pragma unroll
            for (int h = 0; h < JG / 2; ++h) av4[h] = *reinterpret_cast<const uint4*>(smem + abase + 16 * h);
            int4 sqv = make_int4(0, 0, 0, 0);
            if (BITS == 4) sqv = *reinterpret_cast<const int4*>(sq_l + me * lay.sa_pitch + (c - coff) * 4);
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
    if constexpr (SPLIT) {
        // The chain wave's ticket says whether this workgroup folds.
        lds_barrier();
        if (!*reinterpret_cast<const int*>(smem + split_flag_off(a.M, a.nblk4, lay.total))) return;
        split_stage();
        lds_barrier();
    }
}

template <int BITS, bool HP, bool FUSED, bool EXTRA, int R, int FUSE, bool P64>
hipError_t launch_dec_t(bool* attr_set, const GemvArgs& a, int grid, int lds, hipStream_t st) {
    auto kern = dec_kernel<BITS, HP, FUSED, EXTRA, R, FUSE, P64>;
    const int key = (BITS == 8 ? 1 : 0) | (HP ? 2 : 0) | (FUSED ? 4 : 0) | (EXTRA ? 8 : 0) | ((R / 2 - 1) << 4) |
                    (P64 ? 32 : 0) | FUSE << 6;
    if (!attr_set[key]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
        if (e != hipSuccess) return e;
        attr_set[key] = true;
    }
    const void* act = FUSED ? static_cast<const void*>(a.A) : static_cast<const void*>(a.Aq);
    const int npw = (a.nbg + kProducers - 1) / kProducers;
    const int misc = a.sc_shift | (a.RS == 1 ? 2 : a.RS == 2 ? 1 : 0) << 5 | a.RG << 8 | a.pair_xcd << 12 | npw << 16;
    const int base_t = a.ntiles / a.NG, rem_t = FUSE == kFuseSplit ? a.split : a.ntiles - base_t * a.NG;
    kern<<<grid, kDecWaves * 64, lds, st>>>(act, a.W, a.S, base_t, a.nblk, a.M, a.nbg, rem_t, a.NG, a.ngrp, misc, a);
    return hipGetLastError();
}

template <int BITS, bool HP, bool FUSED, bool EXTRA, bool P64>
hipError_t launch_dec_w(bool* attr_set, const GemvArgs& a, int grid, int lds, int fuse, hipStream_t st) {
    if (fuse == kFusePair)
        return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFusePair, P64>(attr_set, a, grid, lds, st);
    if (fuse == kFusePairFlow)
        return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFusePairFlow, P64>(attr_set, a, grid, lds, st);
    if (fuse == kFusePairFlowStream)
        return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFusePairFlowStream, P64>(attr_set, a, grid, lds, st);
    if (fuse == kFuseSplit) {
        if constexpr (FUSED) return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFuseSplit, P64>(attr_set, a, grid, lds, st);
        return hipErrorInvalidValue;  // split pieces quantize in the prologue
    }
    if (fuse == kFuseStream)
        return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFuseStream, P64>(attr_set, a, grid, lds, st);
    if (fuse == kFuseFlow)
        return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFuseFlow, P64>(attr_set, a, grid, lds, st);
    if (fuse == kFuseFlowStream)
        return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFuseFlowStream, P64>(attr_set, a, grid, lds, st);
    if constexpr (!EXTRA) {
        if (fuse == kFuseMulti)
            return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFuseMulti, P64>(attr_set, a, grid, lds, st);
        if constexpr (FUSED) {
            if (fuse == kFuseNormMulti)
                return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFuseNormMulti, P64>(attr_set, a, grid, lds, st);
        } else if (fuse == kFuseNormMulti) {
            return hipErrorInvalidValue;  // the host normalizes first when the prologue does not quantize
        }
    } else if (fuse >= kFuseMulti) {
        return hipErrorInvalidValue;  // the host sends per-block-metadata handles one by one
    }
    return launch_dec_t<BITS, HP, FUSED, EXTRA, kDecRing, kFusePlain, P64>(attr_set, a, grid, lds, st);
}

template <int BITS, bool HP, bool FUSED, bool EXTRA>
hipError_t launch_dec_r(bool* attr_set, const GemvArgs& a, int grid, int lds, int fuse, bool p64,
                        hipStream_t st) {
    return p64 ? launch_dec_w<BITS, HP, FUSED, EXTRA, true>(attr_set, a, grid, lds, fuse, st)
               : launch_dec_w<BITS, HP, FUSED, EXTRA, false>(attr_set, a, grid, lds, fuse, st);
}

template <int BITS, bool HP>
hipError_t launch_dec_bits(bool* attr_set, const GemvArgs& a, int grid, int lds, int fuse, bool p64, bool fused,
                           bool extra, hipStream_t st) {
    if (extra) return fused ? launch_dec_r<BITS, HP, true, true>(attr_set, a, grid, lds, fuse, p64, st)
                            : launch_dec_r<BITS, HP, false, true>(attr_set, a, grid, lds, fuse, p64, st);
    return fused ? launch_dec_r<BITS, HP, true, false>(attr_set, a, grid, lds, fuse, p64, st)
                 : launch_dec_r<BITS, HP, false, false>(attr_set, a, grid, lds, fuse, p64, st);
}

}  // namespace bq

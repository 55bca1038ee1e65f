// prefill_kernel.h -- the prefill GEMM (rows past the decode kernel's) and its launcher,
// instantiated per (bits, activation mode) by pf_w{4,8}_{hp,lp}.hip.
#pragma once

#include "qmm_common.h"

namespace bq {

template <int BITS, bool HP, int SCM, int CT, int RP, int S>
__global__ __launch_bounds__(kPfWaves * 64) void prefill_kernel(PfArgs a) {
    using L = PfLayout<CT, SCM, BITS, RP, S>;
    static_assert(S == 2 || S == 3, "ring depth");
    extern __shared__ __align__(16) char pf_lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int col = lane & 15, grp = lane >> 4;
    // Wave w: row pair w % RP (two 16-row tiles) and column part w / RP of
    // the kParts parts; waves w and w + 4 share a SIMD.
    constexpr int kParts = kPfWaves / RP;
    static_assert(kPfWaves % RP == 0 && CT >= kParts, "every part holds a tile");
    const int rp = wave % RP, part = wave / RP;
    // Part q: tiles [q CTB + min(q, CTR), ...), CTB + 1 of them for q < CTR.
    constexpr int CTB = CT / kParts, CTR = CT % kParts;
    const int part_t0 = part * CTB + min(part, CTR), part_nt = CTB + (part < CTR ? 1 : 0);
    const int t0 = blockIdx.x * CT;
    const int rt0 = blockIdx.y * (2 * RP) + 2 * rp;
    const bool active = rt0 * 16 < a.M;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(pf_lds));
    const int nch = a.nch;
    const int nst = (nch + kPfChunks - 1) / kPfChunks;
    const bool odd = a.nblk & 1;

    // Shared part of a chunk (INT8) or stage (INT4).
    // INT8: loads k < kWJ load weight tile min(wave + kPfWaves k, CT - 1)
    // (a spare load repeats the last tile: same bytes, same place).  Loads
    // k >= kWJ load the 1 KB of sums and scales at x0 = kWS + 1024 u,
    // u = (k - kWJ) * kPfWaves + wave (clamped), lane bytes x0 + 16*lane.
    // INT4: slot k loads unit u = k * kPfWaves + wave (clamped): raw tile u
    // of the stage into chunk 0's weight area, or KB u - CT of the raw area.
    const char* src0[L::kPerWave];
    uint32_t step[L::kPerWave], gstep[L::kPerWave], x0s[L::kPerWave];
    bool to_raw[L::kPerWave];
#pragma unroll
    for (int k = 0; k < L::kPerWave; ++k) {
        const int u = BITS == 8 ? min((k - L::kWJ) * kPfWaves + wave, L::kSU - 1)
                                : min(k * kPfWaves + wave, L::kUnits - 1);
        const int x0 = BITS == 8 ? L::kWS + u * 1024 : u * 1024;
        const int x = x0 + 16 * lane;
        x0s[k] = (uint32_t)x0;
        gstep[k] = 0;
        step[k] = 0;
        src0[k] = a.W;
        to_raw[k] = false;
        if (BITS == 8 && k < L::kWJ) continue;
        if (BITS == 4) {
            if (u < CT) {
                const int tc = min(t0 + u, a.ntiles - 1);
                src0[k] = a.W + (size_t)tc * a.nbg * 1024 + 16 * lane;
                step[k] = 1024;
                x0s[k] = (uint32_t)(u * 1024);
            } else {
                const int y = (u - CT) * 1024 + 16 * lane;
                to_raw[k] = true;
                x0s[k] = (uint32_t)((u - CT) * 1024);  // within the stage's raw area
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
    // The workgroup's 2 RP activation records per chunk, 3 DMA units each
    // (bytes 0 and 1024 and the tail from 1152; the last two overlap), split
    // over the waves: unit wave + 8 i, clamped, so a spare slot repeats the
    // last unit's load (same bytes to the same place).
    constexpr int kRecUnits = 6 * RP, kRecPerWave = (kRecUnits + kPfWaves - 1) / kPfWaves;
    const char* rec0 = a.R + (size_t)blockIdx.y * (2 * RP) * nch * kRecBytes;
    uint32_t rec_src[kRecPerWave], rec_dst[kRecPerWave];
#pragma unroll
    for (int i = 0; i < kRecPerWave; ++i) {
        const int u = min(wave + kPfWaves * i, kRecUnits - 1), r = u / 3, pt = u % 3;
        const int off = pt == 0 ? 0 : pt == 1 ? 1024 : 1152;
        rec_src[i] = (uint32_t)(r * nch * kRecBytes + off);
        rec_dst[i] = (uint32_t)(L::kA + r * kRecBytes + off);
    }

    // Load d of this wave's kDmaChunk loads of chunk c into the chunk region
    // at LDS address cbase: the shared slots, then its record units.
    constexpr int kDmaChunk = L::kPerWave + kRecPerWave;
    // INT4: only chunk 0 of a stage (first) carries the stage's shared loads;
    // raw is the LDS address of the stage's raw area.
    auto dma_slot = [&](int c, uint32_t cbase, int d, bool first, uint32_t raw) __attribute__((always_inline)) {
        if (d < L::kPerWave) {
            if (BITS == 8 && d < L::kWJ) {
                const int tile = min(d * kPfWaves + wave, CT - 1);
                const int tc = min(t0 + tile, a.ntiles - 1);
                dma16s(a.W + ((size_t)tc * nch + c) * 1024, 16 * lane, cbase + (uint32_t)(tile * 1024));
            } else if (BITS == 8) {
                const size_t g = SCM == 1 ? (size_t)((2 * c) >> a.sc_shift) : 0;
                dma16(src0[d] + (size_t)c * step[d] + g * gstep[d], cbase + x0s[d]);
            } else if (first) {
                const int sg = c >> 1;
                const size_t g = SCM == 1 ? (size_t)((4 * sg) >> a.sc_shift) : 0;
                dma16(src0[d] + (size_t)sg * step[d] + g * gstep[d], (to_raw[d] ? raw : cbase) + x0s[d]);
            }
        } else {
            const int e = d - L::kPerWave;
            dma16s(rec0 + rec_src[e] + (size_t)c * kRecBytes, 16 * lane, cbase + rec_dst[e]);
        }
    };
    // Raw area of stage g (INT4).
    auto raw_base = [&](int g) { return lds0 + (uint32_t)(L::kRawOff + (g % L::kNRaw) * L::kRaw); };
    // With more than two stages every stage issues the same loads per wave
    // (chunks past the end repeat the last chunk's, into a slot nobody
    // reads), so the wait at a stage's start counts the loads issued after
    // it exactly.  Two stages wait for all loads and skip those chunks (the
    // loads kept the allocator from fitting the widest shapes' registers).
    constexpr int kStageLoads = BITS == 8 ? kPfChunks * kDmaChunk : kDmaChunk + (kPfChunks - 1) * kRecPerWave;
    auto issue_stage = [&](int g, int buf) __attribute__((always_inline)) {
        const uint32_t sbase = lds0 + (uint32_t)(buf * L::kStage);
#pragma unroll
        for (int cc = 0; cc < kPfChunks; ++cc) {
            const int c = min(g * kPfChunks + cc, nch - 1);
            if (S == 2 && g * kPfChunks + cc >= nch) continue;
#pragma unroll
            for (int d = 0; d < kDmaChunk; ++d) dma_slot(c, sbase + (uint32_t)(cc * L::kChunk), d, cc == 0, raw_base(g));
        }
    };

    // INT4: expands stage g (buffer buf) in place from its raw area (with more
    // than one row pair all threads share the tiles and a workgroup barrier
    // must follow).  Wave w takes tiles w, w + 8, ... (with one row pair, the
    // tiles of its column part); each lane takes one (column, k-octet) of
    // the tile and writes that octet of the four blocks where pf_w_byte puts
    // it.  The nibble sums of a column's four octets meet across lanes.
    auto expand = [&](int g, int buf) {
        if constexpr (BITS == 4) {
            char* sb = pf_lds + buf * L::kStage;
            const char* raw = pf_lds + L::kRawOff + (g % L::kNRaw) * L::kRaw;
            // Lane l expands octet o of column c of the tile, with
            // c = (l & 7) + 8 ((l >> 4) & 1) and o = ((l >> 3) & 1) + 2 (l >> 5):
            // eight lanes read 128 contiguous raw bytes, and sixteen lanes
            // write 128 contiguous bytes of operands (pf_w_byte), so neither
            // side has bank conflicts.
            const int c = (lane & 7) + 8 * ((lane >> 4) & 1), o = ((lane >> 3) & 1) + 2 * (lane >> 5), cc = o & 1;
            // One row pair: each wave expands the tiles of its own column
            // part, which no other wave reads, so no barrier has to follow.
            const int t_beg = RP == 1 ? part_t0 : wave, t_end = RP == 1 ? part_t0 + part_nt : CT;
            const int t_step = RP == 1 ? 1 : kPfWaves;
            for (int t = t_beg; t < t_end; t += t_step) {
                const int wl = t * 1024 + 16 * (c + 16 * o);
                const uint4 w = *reinterpret_cast<const uint4*>(sb + wl);
                const uint32_t z = SCM == 2 ? *reinterpret_cast<const uint32_t*>(raw + L::kRawZ + t * 64 + 4 * c)
                                            : 0x08080808u;
                const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
                uint32_t lo[4], hi[4], nsum[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    // b = n - zp as a signed byte: n + (128 - zp), then flip
                    // the top bit.  zp is a signed byte in [-112, 127]
                    // (i4_prepack sends lower legacy zero points to the INT8
                    // representation), so 128 - zp is in [1, 240] and
                    // n + 128 - zp in [1, 255]: no carry crosses a byte.
                    const int zs = SCM == 2 ? (int)(int8_t)(z >> (8 * b)) : 8;
                    const uint32_t zr = (uint32_t)(128 - zs) * 0x01010101u;
                    lo[b] = ((wv[b] & 0x0F0F0F0Fu) + zr) ^ 0x80808080u;
                    hi[b] = (((wv[b] >> 4) & 0x0F0F0F0Fu) + zr) ^ 0x80808080u;
                    nsum[b] = __builtin_amdgcn_udot8(wv[b], 0x11111111u, 0u, false);  // <= 120
                }
                // Octet o of blocks 0-3 (chunk b >> 1, block b & 1) into the
                // operand order; this wave alone reads and writes tile t,
                // and all of its reads of t are done (the writes use them).
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    *reinterpret_cast<uint2*>(sb + (b >> 1) * L::kChunk + t * 1024 + pf_w_byte(4, c, o, b & 1)) =
                        make_uint2(lo[b], hi[b]);
                // Per-column nibble sums of blocks (0, 1) and (2, 3), two per
                // dword, summed over the four octets: lanes l, l ^ 32 (o ^ 2)
                // by a half swap, then l ^ 8 (o ^ 1) by a row rotate of 8.
                uint32_t ps[2] = {nsum[0] | nsum[1] << 16, nsum[2] | nsum[3] << 16};
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const auto s32 = __builtin_amdgcn_permlane32_swap(ps[q], ps[q], false, false);
                    const uint32_t y = s32[0] + s32[1];
                    ps[q] = y + (uint32_t)__builtin_amdgcn_update_dpp(0, (int)y, 0x128, 0xF, 0xF, false);
                }
                char* cb = sb + cc * L::kChunk;
                if (o < 2) {
                    // Row o: 128 * sum(n - zp) of chunk o's two blocks.
                    const uint32_t p2 = cc ? ps[1] : ps[0];
                    const uint32_t zz = SCM == 2 ? z >> (16 * cc) : 0x0808u;
                    const int s0 = (int)(p2 & 0xFFFFu) - 32 * (int)(int8_t)zz;
                    const int s1 = (int)(p2 >> 16) - 32 * (int)(int8_t)(zz >> 8);
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
    // Lane l: A row / output column c32 = l & 31, k half kh = l >> 5.  The A
    // operand is one 16-byte LDS read: records hold k-octets 2 kh and
    // 2 kh + 1 of a row side by side (pf_rec_byte).  So do expanded INT4
    // tiles for B; INT8 tiles hold octet o of both blocks side by side, and
    // B takes two 8-byte halves 256 bytes apart (pf_w_byte).  Reading those
    // with one ds_read2_b64 straight into the operand was slower than the
    // register moves after a merged 16-byte read: an 8-byte access at a
    // 16-byte lane stride uses half the LDS banks.
    auto run32 = [&](auto ctw_tag, int toff) {
        constexpr int CTW = decltype(ctw_tag)::value;
        constexpr int NG = CTW / 2;
        constexpr int NG1 = NG > 0 ? NG : 1;  // array extents (a part of one tile has no group)
        constexpr bool ODD = (CTW & 1) != 0;
        const int c32 = lane & 31, kh = lane >> 5;
        float sbg[NG1], sbo = 0.0f;
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
        float acc[NG1][16], acco[2][4];
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[g][j] = 0.0f;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acco[r][i] = 0.0f;

        // dma_tag: 0 no loads, 1 or 2 the loads of chunk 0 or 1 of the stage
        // S - 1 ahead (chunk c_next, at LDS nbase; nraw: that buffer's raw
        // area).
        auto compute = [&](const char* cp, auto nb_tag, auto dma_tag, int c_next, uint32_t nbase, uint32_t nraw) {
            constexpr int NB = decltype(nb_tag)::value;
            constexpr bool DMA = decltype(dma_tag)::value != 0;
            constexpr bool BOTH = decltype(dma_tag)::value == 3;  // both chunks of the next stage
            constexpr bool FIRST = decltype(dma_tag)::value == 1 || BOTH;
            const int c_next2 = min(c_next + 1, nch - 1);
            constexpr int kAhead = 1;            // groups read ahead
            constexpr int NGB = NG * NB;         // group steps
            constexpr int NS = NGB + (ODD ? NB : 0);
            constexpr int TL = DMA ? (BOTH ? 2 : 1) * kDmaChunk : 0;  // loads this call issues
            const char* ar = cp + L::kA + 2 * rp * kRecBytes;
            v4i a_h[2], a_l[2];
            float sa[2][16];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const char* rb = ar + (c32 >> 4) * kRecBytes + b * 1024 + pf_rec_byte(c32 & 15, 2 * kh);
                a_h[b] = *reinterpret_cast<const v4i*>(rb);
                a_l[b] = *reinterpret_cast<const v4i*>(rb + 512);
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
            uint64_t ah[2][2], al[2][2], bwo[2] = {0, 0};
            float so[2][2][4];
            int2 wso = make_int2(0, 0);
            float sbo2[2] = {0.0f, 0.0f};
            auto load_odd = [&]() {
                if (!ODD) return;
#pragma unroll
                for (int r = 0; r < 2; ++r)
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        const char* q = ar + r * kRecBytes + b * 1024 + pf_rec_byte(col, grp);
                        ah[r][b] = *reinterpret_cast<const uint64_t*>(q);
                        al[r][b] = *reinterpret_cast<const uint64_t*>(q + 512);
                        const float4 s4 = *reinterpret_cast<const float4*>(ar + r * kRecBytes + kRecA + b * 64 + 16 * grp);
                        so[r][b][0] = s4.x;
                        so[r][b][1] = s4.y;
                        so[r][b][2] = s4.z;
                        so[r][b][3] = s4.w;
                    }
                const int t = toff + CTW - 1;
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    bwo[b] = *reinterpret_cast<const uint64_t*>(cp + t * 1024 + pf_w_byte(BITS, col, grp, b));
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
            v4i bq[NG1][2];  // B operand per group and block
            int2 wsg[NG1];
            float sbv[NG1][2];
            auto load_group = [&](int g) {
                if (g >= NG) return;
                const int t = toff + 2 * g + (c32 >> 4);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    if (BITS == 8) {
                        const char* bp = cp + t * 1024 + pf_w_byte(8, c32 & 15, 2 * kh, b);
                        const uint2 lo = *reinterpret_cast<const uint2*>(bp);
                        const uint2 hi = *reinterpret_cast<const uint2*>(bp + 256);
                        bq[g][b] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
                    } else {
                        bq[g][b] = *reinterpret_cast<const v4i*>(cp + t * 1024 + pf_w_byte(4, c32 & 15, 2 * kh, b));
                    }
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
            auto bopo = [&](int b) -> uint64_t { return bwo[b]; };
            v16i h32[NGB > 0 ? NGB : 1], d32[NGB > 0 ? NGB : 1];
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
                // Load e of the TL this call issues goes out at step
                // e NS / TL: evenly over the steps.
#pragma unroll
                for (int e = 0; e < TL; ++e) {
                    if (e * NS / TL != s) continue;
                    if (e < kDmaChunk) dma_slot(c_next, nbase, e, FIRST, nraw);
                    else dma_slot(c_next2, nbase + (uint32_t)L::kChunk, e - kDmaChunk, false, nraw);
                }
                step_h(s + 1);
                step_e(s);
                step_d(s + 1);
                __builtin_amdgcn_sched_barrier(0);
            }

        };

        static_assert(kPfChunks == 2, "stage loop");
        constexpr std::integral_constant<int, 2> two{};
        constexpr std::integral_constant<int, 1> one{};
        constexpr std::integral_constant<int, 1> dma0{};
        constexpr std::integral_constant<int, 2> dma1{};
        constexpr std::integral_constant<int, 0> no_dma{};
        constexpr std::integral_constant<int, 3> dma01{};
        // Ring of S stage buffers: stage g lives in buffer g % S.  The first
        // S - 1 stages are issued up front; computing stage g issues stage
        // g + S - 1 (chunks clamped to the last one).  At the start of stage
        // g the loads of the stages after it that are already issued may
        // stay in flight.
        issue_stage(0, 0);
        if (S > 2) issue_stage(1, 1);
        for (int g = 0; g + 1 < nst; ++g) {
            const int ahead = min(g + S - 2, nst - 1) - g;  // stages issued after g (uniform)
            if (S > 2 && ahead > 0) __builtin_amdgcn_s_waitcnt(vm_wait(kStageLoads));
            else __builtin_amdgcn_s_waitcnt(vm_wait(0));
            lds_barrier();
            const int buf = g % S;
            if (BITS == 4) {
                expand(g, buf);
                if (RP > 1) lds_barrier();
                else asm volatile("" ::: "memory");
            }
            const int gn = g + S - 1, bn = gn % S;  // stage issued now, and its buffer
            const uint32_t nbase = lds0 + (uint32_t)(bn * L::kStage);
            const int cn = min(gn * kPfChunks, nch - 1);
            // With two stages gn = g + 1 < nst always: a straight-line body
            // (a branch here makes the allocator copy the accumulators).
            if (S == 2 || gn < nst) {
                if (active) {
                    const char* sp = pf_lds + buf * L::kStage;
                    if (S == 2) {
                        // Both chunks' loads during the first chunk: the
                        // second chunk's have a whole chunk to land.
                        compute(sp, two, dma01, cn, nbase, raw_base(gn));
                        compute(sp + L::kChunk, two, no_dma, 0, 0u, 0u);
                    } else {
                        compute(sp, two, dma0, cn, nbase, raw_base(gn));
                        compute(sp + L::kChunk, two, dma1, min(cn + 1, nch - 1), nbase + (uint32_t)L::kChunk,
                                raw_base(gn));
                    }
                } else {
                    issue_stage(gn, bn);
                }
            } else if (S > 2 && active) {
                const char* sp = pf_lds + buf * L::kStage;
                compute(sp, two, no_dma, 0, 0u, 0u);
                compute(sp + L::kChunk, two, no_dma, 0, 0u, 0u);
            }
        }
        __builtin_amdgcn_s_waitcnt(vm_wait(0));
        lds_barrier();
        if (BITS == 4) {
            expand(nst - 1, (nst - 1) % S);
            if (RP > 1) lds_barrier();
            else asm volatile("" ::: "memory");
        }
        if (!active) return;
        {
            const char* sp = pf_lds + ((nst - 1) % S) * L::kStage;
            const int c0 = (nst - 1) * kPfChunks;
            if (c0 + 1 < nch) {
                compute(sp, two, no_dma, 0, 0u, 0u);
                if (odd) compute(sp + L::kChunk, one, no_dma, 0, 0u, 0u);
                else compute(sp + L::kChunk, two, no_dma, 0, 0u, 0u);
            } else if (odd) {
                compute(sp, one, no_dma, 0, 0u, 0u);
            } else {
                compute(sp, two, no_dma, 0, 0u, 0u);
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
    if constexpr (CTR > 0) {
        if (part < CTR) {
            run32(std::integral_constant<int, CTB + 1>{}, part_t0);
            return;
        }
    }
    run32(std::integral_constant<int, CTB>{}, part_t0);
}


template <int BITS, bool HP, int SCM, int CT, int RP, int S>
hipError_t launch_pf_t(bool* pf_attr, const PfArgs& p, dim3 grid, hipStream_t st) {
    using L = PfLayout<CT, SCM, BITS, RP, S>;
    auto kern = prefill_kernel<BITS, HP, SCM, CT, RP, S>;
    int slot = 0;
    while (kPfCfgs[slot].rp != RP || kPfCfgs[slot].ct != CT) ++slot;
    const int key = (HP ? 1 : 0) | SCM << 1 | slot << 3 | (BITS == 4 ? 128 : 0);
    if (!pf_attr[key]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, L::kBytes);
        if (e != hipSuccess) return e;
        pf_attr[key] = true;
    }
    kern<<<grid, kPfWaves * 64, L::kBytes, st>>>(p);
    return hipGetLastError();
}

// One case per entry of kPfCfgs (row pairs, column tiles, ring stages).
template <int BITS, bool HP, int SCM>
hipError_t launch_pf_scm(bool* pf_attr, const PfArgs& p, int rp, int ct, dim3 grid, hipStream_t st) {
    switch (rp * 100 + ct) {
        case 417: return launch_pf_t<BITS, HP, SCM, 17, 4, 2>(pf_attr, p, grid, st);
        case 416: return launch_pf_t<BITS, HP, SCM, 16, 4, 2>(pf_attr, p, grid, st);
        case 413: return launch_pf_t<BITS, HP, SCM, 13, 4, 2>(pf_attr, p, grid, st);
        case 412: return launch_pf_t<BITS, HP, SCM, 12, 4, 2>(pf_attr, p, grid, st);
        case 409: return launch_pf_t<BITS, HP, SCM, 9, 4, 2>(pf_attr, p, grid, st);
        case 408: return launch_pf_t<BITS, HP, SCM, 8, 4, 2>(pf_attr, p, grid, st);
        case 405: return launch_pf_t<BITS, HP, SCM, 5, 4, 2>(pf_attr, p, grid, st);
        case 404: return launch_pf_t<BITS, HP, SCM, 4, 4, 2>(pf_attr, p, grid, st);
        case 216: return launch_pf_t<BITS, HP, SCM, 16, 2, 2>(pf_attr, p, grid, st);
        case 208: return launch_pf_t<BITS, HP, SCM, 8, 2, 3>(pf_attr, p, grid, st);
        case 204: return launch_pf_t<BITS, HP, SCM, 4, 2, 3>(pf_attr, p, grid, st);
        case 116: return launch_pf_t<BITS, HP, SCM, 16, 1, 2>(pf_attr, p, grid, st);
        case 108: return launch_pf_t<BITS, HP, SCM, 8, 1, 3>(pf_attr, p, grid, st);
        default: return hipErrorInvalidValue;
    }
}

template <int BITS, bool HP>
hipError_t launch_pf(bool* pf_attr, const PfArgs& p, int scm, int rp, int ct, dim3 grid, hipStream_t st) {
    if (scm == 2) return launch_pf_scm<BITS, HP, 2>(pf_attr, p, rp, ct, grid, st);
    if (scm == 1) return launch_pf_scm<BITS, HP, 1>(pf_attr, p, rp, ct, grid, st);
    return launch_pf_scm<BITS, HP, 0>(pf_attr, p, rp, ct, grid, st);
}

}  // namespace bq

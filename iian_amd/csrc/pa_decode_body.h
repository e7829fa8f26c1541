// pa_decode_body.h - the f16 paged decode / spec-verify attention of one stream-K
// piece (one wave), shared by the decode kernel (pa_decode.hip) and the
// mixed-batch prefill kernel (pa_prefill.hip), which runs decode workers in
// its trailing workgroups.  The algorithm is described in pa_decode.hip.
#pragma once

#include "pa_common.h"

namespace iian_pa {

// K/V are read once per call: non-temporal loads keep them from evicting the
// block tables and partials.  Measured on MI355X: +5% at D=128 (256-byte head
// slices), -7% at D=256, so it is chosen per head size.  Head pairs at D = 96
// (HG = 2) load cached: a pair's three lines are requested by two load
// instructions each (one per head), and a cached line serves the second
// (Phi-3.5 shapes: 414 against 434 us, HBM traffic 1.12x -> the lines once).
template <int D, int HG = 1>
struct KvStream {
    static constexpr bool kNonTemporal = D <= 128 && HG == 1;
};

template <bool NT, typename T>
__device__ __forceinline__ T stream_load(const T *ptr) {
    if constexpr (NT)
        return __builtin_nontemporal_load(ptr);
    else
        return *ptr;
}

template <int D>
struct KRegs {
    u32x4 k[2][D / 32];
};
template <int D>
struct VRegs {
    uint32_t v[8][D / 32];   // 8 cells x (D/16) halves per lane
};

// K: lane (n, g) loads cells tile + 8*(n/4) + 4h + (n%4), dims 32ks + 8g .. +8
template <int D, bool NT>
__device__ __forceinline__ void load_k(const AttnParams &p, const TableWindow &tw, int L, int hk, int tile,
                                       KRegs<D> &r) {
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int last = L - 1;
    const int grp = min(tile + 8 * (n >> 2), last);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int c = min(tile + 8 * (n >> 2) + 4 * h + (n & 3), last);
        const uint32_t row = table_row(p, tw, grp, c);
        const char *base = p.k_pool + pool_off(row, p.k_row) + (hk * D * 2 + g * 16);
#pragma unroll
        for (int ks = 0; ks < D / 32; ks++) r.k[h][ks] = stream_load<NT>((const u32x4 *) (base + ks * 64));
    }
}

// V: lane (n, g) loads cells tile + 8g + e, dims (D/16)*n .. +D/16
template <int D, bool NT>
__device__ __forceinline__ void load_v(const AttnParams &p, const TableWindow &tw, int L, int hk, int tile,
                                       VRegs<D> &r) {
    constexpr int VW = D / 32;
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int last = L - 1;
    const int grp = min(tile + 8 * g, last);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int c = min(tile + 8 * g + e, last);
        const uint32_t row = table_row(p, tw, grp, c);
        const uint32_t *src = (const uint32_t *) (p.v_pool + pool_off(row, p.v_row) + (hk * D * 2 + n * (D / 8)));
        if constexpr (VW == 2) {
            const u32x2 x = stream_load<NT>((const u32x2 *) src);
            r.v[e][0] = x[0];
            r.v[e][1] = x[1];
        } else if constexpr (VW == 3) {   // head size 96: 12-byte slices, 4-byte aligned
#pragma unroll
            for (int i = 0; i < 3; i++) r.v[e][i] = stream_load<NT>(src + i);
        } else {
#pragma unroll
            for (int i = 0; i < VW; i += 4) {
                const u32x4 x = stream_load<NT>((const u32x4 *) (src + i));
                r.v[e][i] = x[0];
                r.v[e][i + 1] = x[1];
                r.v[e][i + 2] = x[2];
                r.v[e][i + 3] = x[3];
            }
        }
    }
}

// iian_pa_write_attention: the query tokens of a decode sequence are the
// step's new tokens, and token t's K/V rows belong at the cell of its position
// pos[t] (the slot the engine's set_rows writes).  The piece whose tile range
// [cb, ce) holds that cell writes f16(row) (RNE, as iian_pa_kv_write
// converts) for its kv heads at the start of the piece: each (cell, kv head)
// slice lies in exactly one piece of its segment, so every new row is written
// once.  The tile loop waits for the stores (vmcnt(0)) before it loads a tile
// that holds a query position, so this wave reads the new rows back from its
// own XCD's L2; no other segment reads those bytes.  One 16-byte chunk of one
// row per lane and step.
// The row comes from the block table itself (the piece's table window need
// not reach the cell); a row whose block id lies outside the pool is not
// written (bit 0, as iian_pa_kv_write flags a slot it skips).
template <int D, int HG>
__device__ __forceinline__ void write_new_rows(const AttnParams &p, const SeqWindow &w, int s, int cb, int ce,
                                               int hk0) {
    constexpr int CH = D / 8;   // 16-byte chunks per head slice
    const int lane = threadIdx.x & 63;
    const int64_t rk = (int64_t) p.Hkv * D;   // f32 row elements of k_new and v_new
    for (int j = 0; j < w.nq; j++) {
        const int t = w.q0 + j;
        const int ps = p.pos[t];
        if (ps < cb || ps >= ce || ps >= w.L) continue;   // wave-uniform
        const int b = ps >> p.bs_log2;
        const int32_t id = b < p.max_blocks ? p.bt[(int64_t) s * p.max_blocks + b] : -1;
        if ((uint32_t) id >= (uint32_t) p.num_blocks) {
            if (lane == 0 && p.err) atomicOr(p.err, 1);
            continue;
        }
        const uint32_t row = ((uint32_t) id << p.bs_log2) | (uint32_t) (ps & ((1 << p.bs_log2) - 1));
        for (int it = lane; it < 2 * HG * CH; it += 64) {
            const int tv = it / (HG * CH), hk = hk0 + (it / CH) % HG, c = it % CH;
            const float *src = (tv ? p.v_new : p.k_new) + (int64_t) t * rk + hk * D + 8 * c;
            const float4 a = *(const float4 *) src, b = *(const float4 *) (src + 4);
            const u32x4 v = {pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y), pack_f16x2(b.z, b.w)};
            *(u32x4 *) ((char *) (tv ? p.v_pool : p.k_pool) + pool_off(row, p.k_row) + (hk * D * 2 + 16 * c)) = v;
        }
    }
}

// One piece: window tiles [pc.t0, pc.t1) of sequence pc.s at kv head pc.hk.
// FUSED: a split segment is merged by its last piece to finish (arrive_last),
// not by pa_merge_kernel.  LREC (NRT = 1, pa_decode_seg_kernel): the block-
// table window comes loaded (*tw_pre, covering the piece's first tile), and the
// piece's record goes to the wave's LDS record lrec (O rows at lrec[r*D + d],
// (m, l) of row r at lrec[16*D + 2r]) for a merge inside the workgroup.
// HG = 2 (head size 96): the piece covers kv heads 2*pc.hk and 2*pc.hk + 1,
// whose 192-byte slices of a cell row are three whole 128-byte lines, where
// one head's slice shares a line with its neighbour's (one head per wave
// fetched those lines once per head: 4/3 of the bytes).  Row r < 2M of the
// tile is row r % M of head r / M (M <= 8 rows per head); QK^T and PV run once
// per head, each on the other head's rows too, and each lane keeps the head
// of its own row.
template <int D, int NRT, bool FUSED = false, bool LREC = false, int HG = 1, bool WR = false>
__device__ __forceinline__ void decode_piece(const AttnParams &p, const SeqWindow &w, const Piece &pc,
                                             float *lrec = nullptr, const TableWindow *tw_pre = nullptr) {
    static_assert(!LREC || (NRT == 1 && !FUSED), "LDS records hold one 16-row tile");
    static_assert(HG == 1 || (HG == 2 && NRT == 1 && !FUSED && !LREC), "head pairs: one 16-row tile, merge launch");
    constexpr int KS = D / 32;
    constexpr int DPL = D / 16;
    constexpr bool NT = KvStream<D, HG>::kNonTemporal;
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int s = pc.s, hk = pc.hk * HG;   // (first) kv head of the piece
    const int M = w.nq * p.gqa;            // rows per kv head
    // kv head slot (0 or 1) and row within its head of tile row r
    auto row_head = [&](int r) { return HG == 1 ? 0 : (r >= M ? 1 : 0); };
    auto row_in_head = [&](int r) { return HG == 1 ? r : (r >= M ? r - M : r); };
    const int cb = w.c_lo + pc.t0 * kTile;
    const int ce = min(w.c_hi, w.c_lo + pc.t1 * kTile);

    TableWindow tw;
    if constexpr (LREC) tw = *tw_pre;
    else if (cb < ce) table_load(p, s, cb >> p.bs_log2, w.L, tw);

    // Q^T B operands (pre-scaled f16 hi/lo pairs), row positions, running state
    f16x8 qh[NRT][KS], ql[NRT][KS];
    int prow[NRT];
    float m_run[NRT], l_run[NRT];
    f32x4 o[NRT][DPL];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        const int r = rt * 16 + n;
        prow[rt] = w.pmax;
        if (r < HG * M) {
            const int rh = row_in_head(r);
            const int t = w.q0 + rh / p.gqa, h = (hk + row_head(r)) * p.gqa + rh % p.gqa;
            prow[rt] = p.pos[t];
            const float *qp = p.q + ((int64_t) t * p.H + h) * D + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                split_f16x8(*(const float4 *) (qp + 32 * ks), *(const float4 *) (qp + 32 * ks + 4), p.qscale,
                            qh[rt][ks], ql[rt][ks]);
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                qh[rt][ks] = ql[rt][ks] = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
        }
        m_run[rt] = -INFINITY;
        l_run[rt] = 0.f;
#pragma unroll
        for (int m = 0; m < DPL; m++) o[rt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const bool own1 = HG > 1 && row_head(n) == 1;   // this lane's row (column of S^T, row of P) is of head slot 1
    // iian_pa_write_attention: this piece's new rows first; a tile that holds a
    // query position is loaded only after the stores completed
    constexpr bool wr = WR;   // p.k_new is set
    auto new_cells = [&](int t0) { return wr && t0 <= w.pmax && t0 + kTile > w.pmin; };
    // (when the first tile holds none, its loads go out before the rows are
    // read and stored, so that round trip overlaps the tile's)
    const bool first_new = cb < ce && new_cells(cb);
    if constexpr (WR) {
        if (first_new) write_new_rows<D, HG>(p, w, s, cb, ce, hk);
        // a new token whose position is not a cell of its sequence is not
        // written either (bit 0); the segment's first piece at kv head 0 says so
        if (pc.t0 == 0 && hk == 0 && p.err)
            for (int j = 0; j < w.nq; j++) {
                const int ps = p.pos[w.q0 + j];
                if ((ps < 0 || ps >= w.L) && lane == 0) atomicOr(p.err, 1);
            }
    }
    if (cb < ce) {
        if (first_new) __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
        KRegs<D> kr[HG];
        VRegs<D> vr[HG];
#pragma unroll
        for (int i = 0; i < HG; i++) load_k<D, NT>(p, tw, w.L, hk + i, cb, kr[i]);
#pragma unroll
        for (int i = 0; i < HG; i++) load_v<D, NT>(p, tw, w.L, hk + i, cb, vr[i]);
        if constexpr (WR)
            if (!first_new) write_new_rows<D, HG>(p, w, s, cb, ce, hk);
        for (int tile = cb; tile < ce; tile += kTile) {
            const int next = tile + kTile;
            const bool has_next = next < ce;
            if (has_next && ((min(next + kTile - 1, w.L - 1) >> p.bs_log2) - tw.first) >= 64)
                table_load(p, s, next >> p.bs_log2, w.L, tw);   // pieces longer than 64 blocks

            // S^T = K Q^T for every row tile (per kv head slot; a lane keeps
            // the scores of its own row's head)
            f32x4 sacc[NRT][2];
#pragma unroll
            for (int rt = 0; rt < NRT; rt++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    f32x4 acc[HG];
#pragma unroll
                    for (int i = 0; i < HG; i++) {
                        acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int ks = 0; ks < KS; ks++) {
                            const f16x8 a = __builtin_bit_cast(f16x8, kr[i].k[h][ks]);
                            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[rt][ks], acc[i], 0, 0, 0);
                            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[rt][ks], acc[i], 0, 0, 0);
                        }
                    }
                    sacc[rt][h] = acc[0];
                    if constexpr (HG > 1) {
#pragma unroll
                        for (int e = 0; e < 4; e++) sacc[rt][h][e] = own1 ? acc[HG - 1][e] : acc[0][e];
                    }
                }
            if (has_next && new_cells(next)) __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the new rows are stored
            if (has_next)
#pragma unroll
                for (int i = 0; i < HG; i++) load_k<D, NT>(p, tw, w.L, hk + i, next, kr[i]);

            // online softmax; P becomes the A operand of PV
            const bool full = tile + kTile <= w.L && (!p.causal || tile + kTile - 1 <= w.pmin) &&
                              (p.n_swa <= 0 || w.pmax - tile < p.n_swa);
            f16x8 pa[NRT];
#pragma unroll
            for (int rt = 0; rt < NRT; rt++) {
                float sv[8];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    sv[i] = sacc[rt][0][i];
                    sv[4 + i] = sacc[rt][1][i];
                }
                if (p.softcap > 0.f) {
#pragma unroll
                    for (int e = 0; e < 8; e++) sv[e] = p.softcap * tanhf(sv[e] * p.softcap_inv) * kLog2e;
                }
                if (!full) {
                    const CellWindow cw = cell_window(tile + 8 * g, 8, w.L, prow[rt], p.causal, p.n_swa);
#pragma unroll
                    for (int e = 0; e < 8; e++) sv[e] = cell_visible(cw, e) ? sv[e] : -INFINITY;
                }
                float mt = sv[0];
#pragma unroll
                for (int e = 1; e < 8; e++) mt = fmaxf(mt, sv[e]);
                mt = wave_max(mt);
                const float mnew = fmaxf(m_run[rt], mt);
                float alpha = 1.f;
                float pv[8];
                if (mnew == -INFINITY) {
#pragma unroll
                    for (int e = 0; e < 8; e++) pv[e] = 0.f;
                } else {
                    alpha = __builtin_amdgcn_exp2f(m_run[rt] - mnew);
#pragma unroll
                    for (int e = 0; e < 8; e++) pv[e] = __builtin_amdgcn_exp2f(sv[e] - mnew);
                }
                m_run[rt] = mnew;
                float ps = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) ps += pv[e];
                l_run[rt] = l_run[rt] * alpha + ps;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float a = __shfl(alpha, 4 * g + i);   // alpha of O row 4g+i
#pragma unroll
                    for (int m = 0; m < DPL; m++) o[rt][m][i] *= a;
                }
                u32x4 pk;
#pragma unroll
                for (int wi = 0; wi < 4; wi++) pk[wi] = pack_f16x2(pv[2 * wi], pv[2 * wi + 1]);
                pa[rt] = __builtin_bit_cast(f16x8, pk);
            }

            // V^T B operands: MFMA m takes dim DPL*n + m of cells 8g .. 8g+7;
            // head slot by head slot, each slot's next V loads reusing its
            // registers as soon as its operands are built.  With head pairs,
            // slot i's PV takes P of slot i's rows only (the A operand row is
            // this lane's row).
            const f16x8 zero = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int i = 0; i < HG; i++) {
                u32x4 vb[DPL];
#pragma unroll
                for (int m = 0; m < DPL; m++) {
                    const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
                    for (int wi = 0; wi < 4; wi++)
                        vb[m][wi] = __builtin_amdgcn_perm(vr[i].v[2 * wi + 1][m >> 1], vr[i].v[2 * wi][m >> 1], sel);
                }
                if (has_next) load_v<D, NT>(p, tw, w.L, hk + i, next, vr[i]);
#pragma unroll
                for (int m = 0; m < DPL; m++)
#pragma unroll
                    for (int rt = 0; rt < NRT; rt++) {
                        const f16x8 pi = HG == 1 ? pa[rt] : ((own1 == (i == 1)) ? pa[rt] : zero);
                        o[rt][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pi, __builtin_bit_cast(f16x8, vb[m]), o[rt][m],
                                                                          0, 0, 0);
                    }
            }
        }
    }

    if (!FUSED && !LREC && pc.t0 == 0 && lane == 0) p.seg_info[pc.seg] = make_int2(pc.rec, pc.pieces);
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        float l = l_run[rt];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if (pc.pieces == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = rt * 16 + 4 * g + i;
                const float lr = __shfl(l, 4 * g + i);
                if (r < HG * M) {
                    const int rh = row_in_head(r);
                    const int t = w.q0 + rh / p.gqa, h = (hk + row_head(r)) * p.gqa + rh % p.gqa;
                    const float inv = lr > 0.f ? 1.f / lr : 0.f;
                    float *op = p.out + ((int64_t) t * p.H + h) * D + DPL * n;
                    if constexpr (DPL % 4 == 0) {
#pragma unroll
                        for (int m = 0; m < DPL; m += 4)
                            *(float4 *) (op + m) = make_float4(o[rt][m][i] * inv, o[rt][m + 1][i] * inv,
                                                               o[rt][m + 2][i] * inv, o[rt][m + 3][i] * inv);
                    } else {   // head size 96: 6 dims per lane, 8-byte aligned
#pragma unroll
                        for (int m = 0; m < DPL; m += 2)
                            *(float2 *) (op + m) = make_float2(o[rt][m][i] * inv, o[rt][m + 1][i] * inv);
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = rt * 16 + 4 * g + i;
                if (r < HG * M) {
                    float *op = LREC ? lrec + r * D + DPL * n : rec_o(p, pc.rec, 0, r, D) + DPL * n;
                    if constexpr (FUSED) {
#pragma unroll
                        for (int m = 0; m < DPL; m += 2) store_pair_agent(op + m, o[rt][m][i], o[rt][m + 1][i]);
                    } else if constexpr (DPL % 4 == 0) {
#pragma unroll
                        for (int m = 0; m < DPL; m += 4)
                            *(float4 *) (op + m) =
                                make_float4(o[rt][m][i], o[rt][m + 1][i], o[rt][m + 2][i], o[rt][m + 3][i]);
                    } else {
#pragma unroll
                        for (int m = 0; m < DPL; m += 2) *(float2 *) (op + m) = make_float2(o[rt][m][i], o[rt][m + 1][i]);
                    }
                }
            }
            const int r = rt * 16 + n;
            if (g == 0 && r < HG * M) {
                if constexpr (FUSED)
                    store_pair_agent(rec_ml(p, pc.rec, 0, r), m_run[rt], l);
                else if constexpr (LREC)
                    *(float2 *) (lrec + 16 * D + 2 * r) = make_float2(m_run[rt], l);
                else
                    *(float2 *) rec_ml(p, pc.rec, 0, r) = make_float2(m_run[rt], l);
            }
        }
    }
    if constexpr (FUSED) {
        if (pc.pieces > 1 && arrive_last(p.seg_ctr + pc.seg, p.epoch, pc.pieces))
            for (int row0 = 0; row0 < M; row0 += 16) merge_tile16<D>(p, pc.rec0, pc.pieces, 0, row0, M, w.q0, hk);
    }
}

}  // namespace iian_pa

// pa_decode_q8.hip - stream-K paged decode / spec-verify attention over ggml
// Q8_0 KV pools for gfx950 (wave64, MFMA f16).
//
// Pool rows are the reference's Q8_0 rows (ggml-common.h:251-256): a head
// slice is D/32 blocks of {f16 d, int8 q[32]} = 34*D/32 bytes, only 2-byte
// aligned inside the row, so it cannot feed MFMA operands straight from
// memory.  Workers are groups of Hkv workgroups, one per kv head; group g takes
// an equal range of the call's (sequence, 32-cell tile) line (for_each_piece,
// pa_common.h) and each of its workgroups attends that range for its kv head.
// A workgroup has one wave per 16-row query tile (NW = 1, or 2 for
// spec-verify batches of up to 32 rows per kv head).  Each 32-cell tile is
// staged once per workgroup:
//
//   raw load   2 lanes per cell, each loads its half of the cell's K or V head
//              slice as an aligned dword window (issued one tile ahead); with
//              two waves, wave 0 loads K and wave 1 loads V
//   stage      int8 -> f16 is exact (|q| <= 128): bias to unsigned, v_perm the
//              byte under 0x64 (the f16 1024 + u), v_pk_add_f16 -1152.  The
//              f16 rows go to LDS, the block scales d to LDS as f32.
//   QK^T       one v_mfma_f32_16x16x32_f16 per Q8_0 block (k-step = block),
//              scaled by the K block's d per cell in fp32 afterwards
//   PV         V staged as f16(q*d), the correctly rounded dequantised
//              value (both factors exact in f16); V^T operands via
//              ds_read_b64_tr_b16
//
// So K enters the scores as q*d (ggml-quants.c:553-567) with q and d exact and
// the product in fp32, as in the reference's dequantised path; V enters as
// f16(q*d), rounded once as P is.
//
// Memory order: a head slice is 34*D/32 bytes, so the slices of neighbouring
// kv heads share cache lines.  The workgroups of one group are therefore
// dispatched back to back onto one XCD (workgroup id mod 8 selects the XCD),
// and the loads are ordinary cached loads, so a shared line comes from HBM
// once and is then hit in that XCD's L2.
//
// Partial records (one per piece, all kv heads of the group) and the merge are
// shared with pa_decode.hip.
// Semantics follow paged_attn_impl (src/iian/paged_attn.cpp:90-146) run on the
// dequantised pool (the reference CPU op reaches Q8_0 KV only that way).
#include "pa_common.h"
#include "pa_launch.h"

namespace iian_pa {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_q8;

template <int D>
struct Q8Shape {
    static constexpr int NB = D / 32;                       // Q8_0 blocks per head slice
    static constexpr int HS = NB * 34;                      // head-slice bytes
    static constexpr int NBL = NB / 2;                      // blocks staged by one lane (2 lanes per cell)
    static constexpr int SH_MAX = (NB == 2) ? 2 : 0;        // lane slices start 4-aligned unless NB == 2
    static constexpr int W = (34 * NBL + SH_MAX + 3) / 4;   // dwords of one lane's load window
    // LDS rows of f16 values: unpadded with XOR-swizzled chunks at D >= 128
    // (q8_k_off, q8_v_off), padded by 16 bytes at D = 64
    static constexpr bool SWZ = D >= 128;
    static constexpr int STRIDE = SWZ ? D * 2 : D * 2 + 16;
    static constexpr int TILE_BYTES = kTile * STRIDE;
};

// LDS tile layouts at D >= 128, for 64 banks of 4 bytes: a 16-lane b128
// access and a 32-lane b64 access each cover one 256-byte bank window, and a
// row is a whole number of windows.  The staging lanes hold cell l/2, blocks
// (l%2)*NB/2 .. +NB/2 (q8_load_raw).
//
// K: 16-byte chunk c (dims 8c .. 8c+7) of row r sits at chunk
// c ^ swk(r) ^ (c >= 16 ? 8 : 0).  A QK^T read takes one chunk of rows
// 8a + b (+4), a, b < 4, over 16 lanes: swk maps them to 16 distinct
// positions.  A staging write of 16 lanes covers 8 consecutive cells x 2
// halves of the row, and swk takes 8 distinct values in its low three bits
// over 8 aligned cells, while the halves differ in bit 3 (chunk + 8 at
// D = 128; the extra XOR at D = 256, where the halves are 16 chunks apart).
//
// V: 32-byte chunk v (dims 16v .. 16v+15) of row r sits at chunk v ^ swv(r),
// its two 16-byte halves swapped when v >= NB (the chunks the second staging
// lane of a cell writes).  A transpose read of 32 lanes takes one chunk of
// rows {0..3, 8..11} + 4i + 16j: swv maps them to 8 distinct positions.  A
// staging write of 16 lanes (8 cells x 2 lanes, one 16-byte half each) hits
// 8 distinct chunk positions, and the swap puts the two lanes of a cell in
// different halves.
__device__ __forceinline__ int q8_swk(int r) { return (r & 7) ^ (((r >> 3) & 3) << 2); }
__device__ __forceinline__ int q8_swv(int r) { return (r & 3) | ((((r >> 3) ^ (r >> 2)) & 1) << 2); }

// byte offset of 16-byte K chunk c of row r
template <int D>
__device__ __forceinline__ int q8_k_off(int r, int c) {
    if constexpr (Q8Shape<D>::SWZ) return r * Q8Shape<D>::STRIDE + 16 * (c ^ q8_swk(r) ^ (c >= 16 ? 8 : 0));
    else return r * Q8Shape<D>::STRIDE + 16 * c;
}
// byte offset of byte b (0..31) of 32-byte V chunk v of row r
template <int D>
__device__ __forceinline__ int q8_v_off(int r, int v, int b) {
    if constexpr (Q8Shape<D>::SWZ)
        return r * Q8Shape<D>::STRIDE + 32 * (v ^ q8_swv(r)) + (v >= Q8Shape<D>::NB ? b ^ 16 : b);
    else return r * Q8Shape<D>::STRIDE + 32 * v + b;
}

template <int D>
struct Q8Lds {
    __attribute__((aligned(16))) char k[Q8Shape<D>::TILE_BYTES];
    __attribute__((aligned(16))) char v[Q8Shape<D>::TILE_BYTES];
    __attribute__((aligned(16))) float ks[Q8Shape<D>::NB][kTile];
};

// Raw Q8_0 bytes of one tile of one pool: lane l holds blocks [part*NBL,
// part*NBL + NBL) of cell tile + l/2 (part = l%2), as the aligned dword window
// that contains them.  The window never leaves the cell's row: it ends at the
// slice end (NB > 2) or starts at most 2 bytes before the slice (NB == 2).
template <int D>
__device__ __forceinline__ void q8_load_raw(const AttnParams &p, const char *pool, int64_t row_bytes,
                                            const TableWindow &tw, int L, int hk, int tile,
                                            uint32_t (&raw)[Q8Shape<D>::W]) {
    using Q = Q8Shape<D>;
    const int lane = threadIdx.x & 63;
    const int c = min(tile + (lane >> 1), L - 1);
    const uint32_t row = table_row(p, tw, c, c);
    const int off = hk * Q::HS + (lane & 1) * (34 * Q::NBL);
    const uint32_t *src = (const uint32_t *) (pool + pool_off(row, row_bytes) + (off & ~3));
#pragma unroll
    for (int i = 0; i < Q::W; i++) raw[i] = src[i];
}

// Converts a lane's raw window into f16 rows (tile_lds[cell][D]) and f32 block
// scales (sc[block][cell]).  sh = byte offset of the lane's first block in the
// window (0, or 2 for the second lane of a cell when D == 64).  DEQ (V): the
// rows hold f16(q*d), the correctly rounded dequantised value (both factors
// are exact in f16), and no scales are written.
template <int D, bool DEQ>
__device__ __forceinline__ void q8_stage(const uint32_t (&raw)[Q8Shape<D>::W], int sh, char *tile_lds,
                                         float (*sc)[kTile]) {
    using Q = Q8Shape<D>;
    const int lane = threadIdx.x & 63, cell = lane >> 1, part = lane & 1;
#pragma unroll
    for (int j = 0; j < Q::NBL; j++) {
        const int blk = part * Q::NBL + j;
        uint32_t q32[8];
        uint32_t dbits;
        if constexpr (Q::SH_MAX == 0) {
            // the window starts at the lane's first block: block j's scale at
            // byte 34j, its quants at 34j+2 (2 mod 4 for even j, 0 mod 4 for odd)
            const int b0 = 34 * j;
            const int q0 = 34 * j + 2;
            dbits = (raw[b0 >> 2] >> (8 * (b0 & 3))) & 0xffffu;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int i0 = (q0 >> 2) + k;
                q32[k] = (q0 & 3) ? __builtin_amdgcn_alignbyte(raw[min(i0 + 1, Q::W - 1)], raw[i0], q0 & 3) : raw[i0];
            }
        } else {
            // D == 64: one block per lane, starting at byte sh (0 or 2) of the window
            dbits = (raw[0] >> (8 * sh)) & 0xffffu;
#pragma unroll
            for (int k = 0; k < 8; k++)
                q32[k] = sh ? raw[k + 1] : __builtin_amdgcn_alignbyte(raw[k + 1], raw[k], 2);
        }
        const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) dbits);
        if constexpr (!DEQ) sc[blk][cell] = (float) d;
        const f16x2 d2 = {d, d};
        u32x4 h[4];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t lo, hi;
            i8x4_to_f16(q32[k], lo, hi);
            if constexpr (DEQ) {
                lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, lo) * d2);
                hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, hi) * d2);
            }
            h[k >> 1][2 * (k & 1)] = lo;
            h[k >> 1][2 * (k & 1) + 1] = hi;
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int off = DEQ ? q8_v_off<D>(cell, 2 * blk + (k >> 1), 16 * (k & 1)) : q8_k_off<D>(cell, 4 * blk + k);
            *(u32x4 *) (tile_lds + off) = h[k];
        }
    }
}

__device__ __forceinline__ f16x8 lds_tr_b16x8_q8(const char *p0, const char *p1) {
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_q8 *) (uintptr_t) p0);
    const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_q8 *) (uintptr_t) p1);
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 c = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(f16x8, c);
}

// One piece of a group: window tiles [pc.t0, pc.t1) of sequence pc.s at kv
// head pc.hk (workgroup-uniform).
template <int D, int NW>
__device__ __forceinline__ void q8_piece(const AttnParams &p, Q8Lds<D> &lds, const SeqWindow &w, const Piece &pc) {
    using Q = Q8Shape<D>;
    constexpr int NB = Q::NB, NPV = D / 16;
    constexpr int NRAW = NW == 1 ? 2 : 1;   // pools one wave stages: K and V, or one of them
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int s = pc.s, hk = pc.hk;
    const int M = w.nq * p.gqa;
    const int cb = w.c_lo + pc.t0 * kTile;
    const int ce = min(w.c_hi, w.c_lo + pc.t1 * kTile);
    const bool rows_live = wave * 16 < M;   // this wave's row tile holds query rows

    TableWindow tw;
    if (cb < ce) table_load(p, s, cb >> p.bs_log2, w.L, tw);

    // Q^T B operands per block (k-step ks covers dims 32ks .. 32ks+31) as f16
    // hi/lo pairs, row position, state
    f16x8 qh[NB], ql[NB];
    const int qr = wave * 16 + n;
    int prow = w.pmax;
    if (qr < M) {
        const int t = w.q0 + qr / p.gqa, h = hk * p.gqa + qr % p.gqa;
        prow = p.pos[t];
        const float *qp = p.q + ((int64_t) t * p.H + h) * D + 8 * g;
#pragma unroll
        for (int ks = 0; ks < NB; ks++)
            split_f16x8(*(const float4 *) (qp + 32 * ks), *(const float4 *) (qp + 32 * ks + 4), p.qscale, qh[ks],
                        ql[ks]);
    } else {
#pragma unroll
        for (int ks = 0; ks < NB; ks++) qh[ks] = ql[ks] = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
    }
    float m_run = -INFINITY, l_run = 0.f;   // m_run: reference max (log2 units) of O and l
    f32x4 o[NPV];                           // O rows 4g+i, dim 16m + n
#pragma unroll
    for (int m = 0; m < NPV; m++) o[m] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (cb < ce) {
        const bool stage_k = NW == 1 || wave == 0;
        const char *pool0 = stage_k ? p.k_pool : p.v_pool;
        const int64_t row0 = stage_k ? p.k_row : p.v_row;
        const int sh = (Q::SH_MAX == 0) ? 0 : ((hk * Q::HS + (lane & 1) * (34 * Q::NBL)) & 3);
        uint32_t raw[NRAW][Q::W];
        q8_load_raw<D>(p, pool0, row0, tw, w.L, hk, cb, raw[0]);
        if constexpr (NRAW == 2) q8_load_raw<D>(p, p.v_pool, p.v_row, tw, w.L, hk, cb, raw[1]);
        for (int tile = cb; tile < ce; tile += kTile) {
            const int next = tile + kTile;
            const bool has_next = next < ce;
            lds_barrier<NW>();   // every wave is done reading the previous tile
            if (stage_k) q8_stage<D, false>(raw[0], sh, lds.k, lds.ks);   // K: exact int8 values, f32 scales
            else q8_stage<D, true>(raw[0], sh, lds.v, nullptr);          // V: f16(q*d)
            if constexpr (NRAW == 2) q8_stage<D, true>(raw[1], sh, lds.v, nullptr);
            if (has_next && ((min(next + kTile - 1, w.L - 1) >> p.bs_log2) - tw.first) >= 64)
                table_load(p, s, next >> p.bs_log2, w.L, tw);
            if (has_next) {
                q8_load_raw<D>(p, pool0, row0, tw, w.L, hk, next, raw[0]);
                if constexpr (NRAW == 2) q8_load_raw<D>(p, p.v_pool, p.v_row, tw, w.L, hk, next, raw[1]);
            }
            lds_barrier<NW>();   // the staged tile is visible to every wave
            if (!rows_live) continue;

            // S^T = sum_blocks d_K[cell] * (K_int Q^T)
            f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
            // issue priority up for the MFMA clusters (QK^T here, PV below), so
            // that the other wave on the SIMD stages or runs its softmax in
            // their shadow (measured -1.5% at config 4)
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int cr = 8 * (n >> 2) + 4 * h + (n & 3);
#pragma unroll
                for (int ks = 0; ks < NB; ks++) {
                    const f16x8 a = *(const f16x8 *) (lds.k + q8_k_off<D>(cr, 4 * ks + g));
                    const f32x4 dk = *(const f32x4 *) &lds.ks[ks][8 * g + 4 * h];
                    f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[ks], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[ks], c, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) sacc[h][i] = fmaf(c[i], dk[i], sacc[h][i]);
                }
            }

            __builtin_amdgcn_s_setprio(0);
            const bool full = tile + kTile <= w.L && (!p.causal || tile + kTile - 1 <= w.pmin) &&
                              (p.n_swa <= 0 || w.pmax - tile < p.n_swa);
            float sv[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[i] = sacc[0][i];
                sv[4 + i] = sacc[1][i];
            }
            if (p.softcap > 0.f) {
#pragma unroll
                for (int e = 0; e < 8; e++) sv[e] = p.softcap * tanhf(sv[e] * p.softcap_inv) * kLog2e;
            }
            if (!full) {
                const CellWindow cw = cell_window(tile + 8 * g, 8, w.L, prow, p.causal, p.n_swa);
#pragma unroll
                for (int e = 0; e < 8; e++) sv[e] = cell_visible(cw, e) ? sv[e] : -INFINITY;
            }
            float mt = sv[0];
#pragma unroll
            for (int e = 1; e < 8; e++) mt = fmaxf(mt, sv[e]);
            mt = wave_max(mt);
            // Lazy rescale: the reference max only moves when a row's tile max
            // exceeds it by more than kRescaleSlack, so P <= 2^kRescaleSlack
            // and O, l are rescaled only on those (rare, wave-uniform) tiles.
            const bool grow = mt > m_run + kRescaleSlack;
            if (__builtin_amdgcn_ballot_w64(grow)) {
                const float mnew = grow ? mt : m_run;
                const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - mnew) : 1.f;   // 0 when m_run = -inf
                m_run = mnew;
                l_run *= alpha;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float a = __shfl(alpha, 4 * g + i);   // alpha of O row 4g+i
#pragma unroll
                    for (int m = 0; m < NPV; m++) o[m][i] *= a;
                }
            }
            // a row with m_run = -inf has only masked cells so far: its P is 0
            const float mref = m_run == -INFINITY ? 0.f : m_run;
            float pv[8];
            float ps = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                pv[e] = __builtin_amdgcn_exp2f(sv[e] - mref);
                ps += pv[e];
            }
            l_run += ps;

            // O += P V, V staged as f16(q*d)
            const int vr = 8 * g + (n >> 2);   // V rows vr, vr + 4 at byte 8(n%4) of chunk m
            const u32x4 pk = {pack_f16x2(pv[0], pv[1]), pack_f16x2(pv[2], pv[3]), pack_f16x2(pv[4], pv[5]),
                              pack_f16x2(pv[6], pv[7])};
            const f16x8 pb = __builtin_bit_cast(f16x8, pk);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int m = 0; m < NPV; m++) {
                const f16x8 vb = lds_tr_b16x8_q8(lds.v + q8_v_off<D>(vr, m, 8 * (n & 3)),
                                                 lds.v + q8_v_off<D>(vr + 4, m, 8 * (n & 3)));
                o[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pb, vb, o[m], 0, 0, 0);
            }
            __builtin_amdgcn_s_setprio(0);
        }
    }
    if (pc.t0 == 0 && hk == 0 && threadIdx.x == 0) p.seg_info[pc.seg] = make_int2(pc.rec, pc.pieces);
    if (!rows_live) return;

    float l = l_run;
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = wave * 16 + 4 * g + i;
        const float lr = __shfl(l, 4 * g + i);
        if (r >= M) continue;
        if (pc.pieces == 1) {
            const int t = w.q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
            const float inv = lr > 0.f ? 1.f / lr : 0.f;
            float *op = p.out + ((int64_t) t * p.H + h) * D + n;
#pragma unroll
            for (int m = 0; m < NPV; m++) op[16 * m] = o[m][i] * inv;
        } else {
            float *op = rec_o(p, pc.rec, hk, r, D) + n;
#pragma unroll
            for (int m = 0; m < NPV; m++) op[16 * m] = o[m][i];
        }
    }
    if (pc.pieces > 1 && g == 0 && qr < M) *(float2 *) rec_ml(p, pc.rec, hk, qr) = make_float2(m_run, l);
}

// Workgroup b belongs to group g = (b % 8) + 8 * (b / 8 / Hkv) and kv head
// (b / 8) % Hkv, so a group's Hkv workgroups share one XCD (b % 8).
template <int D, int NW>
__global__ __launch_bounds__(64 * NW, (D <= 128) ? 2 : 1) void pa_decode_q8_kernel(AttnParams p) {
    __shared__ Q8Lds<D> lds;
    const int bid = blockIdx.x;
    const int hk = (bid >> 3) % p.Hkv;
    const int grp = (bid & 7) + 8 * ((bid >> 3) / p.Hkv);
    if (grp >= p.sk_workers) return;
    // every wave of the workgroup runs the same (uniform) plan
    for_each_piece<true>(p, grp, hk, [&](const SeqWindow &w, const Piece &pc) { q8_piece<D, NW>(p, lds, w, pc); });
}

template <int D, int NW>
static hipError_t launch_q8_t(const AttnParams &p, hipStream_t stream) {
    const int64_t nwg = 8 * (int64_t) p.Hkv * ((p.sk_workers + 7) / 8);
    if (nwg > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((pa_decode_q8_kernel<D, NW>), dim3((unsigned) nwg), dim3(64 * NW), 0, stream, p);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : launch_merge(p, D, stream);
}

hipError_t launch_decode_q8(const AttnParams &p, int head_dim, hipStream_t stream) {
    const int nw = p.decode_rows > 16 ? 2 : 1;   // as q8_waves_per_wg in pa_abi.hip
    switch (head_dim) {
        case 64: return nw == 1 ? launch_q8_t<64, 1>(p, stream) : launch_q8_t<64, 2>(p, stream);
        case 128: return nw == 1 ? launch_q8_t<128, 1>(p, stream) : launch_q8_t<128, 2>(p, stream);
        case 256: return nw == 1 ? launch_q8_t<256, 1>(p, stream) : launch_q8_t<256, 2>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iian_pa

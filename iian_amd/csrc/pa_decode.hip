// pa_decode.hip - split-K paged decode / spec-verify attention for gfx950 (wave64, MFMA).
//
// One wave per (split, kv head, sequence).  The wave owns every query row of
// its sequence that maps to the kv head: row r = j*gqa + g for query token j
// and head g of the GQA group (so the group shares each K/V load), up to 16*NRT
// rows.  It walks its split's cells in 32-cell tiles straight from the block
// table (no gather), with the next tile's K/V loads in flight while the current
// tile is computed:
//
//   S^T (32 cells x 16 rows) = K * Q^T     v_mfma_f32_16x16x32_f16, K rows are
//                                           the A operand: each lane loads 16
//                                           contiguous bytes of one K row
//   online softmax (exp2 domain)           each lane holds 8 cells of one row;
//                                           row max/sum via xor-16/32 shuffles
//   O (16 rows x D) += P * V               P stays in registers as the A
//                                           operand; V^T B operands are built
//                                           from 16-byte row loads with v_perm
//
// Splits write unnormalised partials (O, m, l); pa_merge combines them with a
// log-sum-exp merge.  A sequence with a single split writes its output directly.
// Semantics follow paged_attn_impl (src/iian/paged_attn.cpp:90-146): masks
// (:124), softcap (:127), all-masked rows -> 0 (:132).
#include "pa_common.h"
#include "pa_launch.h"

namespace iian_pa {

// KV storage formats handled by the tile loader.
enum KvFmt { KV_F16 = 1, KV_Q8_0 = 8 };

template <int D, int KV>
struct TileRegs;

// f16: K half h, k-step ks -> 8 halves; V: 8 cells x (D/16) halves per lane.
template <int D>
struct TileRegs<D, KV_F16> {
    static constexpr int KS = D / 32;
    static constexpr int VW = D / 32;    // dwords of V per cell per lane (D/16 halves)
    u32x4 k[2][KS];
    uint32_t v[8][VW];
};

template <int D>
__device__ __forceinline__ void load_tile_f16(const AttnParams &p, const SeqWindow &w, int s, int hk, int tile,
                                              TileRegs<D, KV_F16> &r) {
    constexpr int KS = D / 32;
    constexpr int VW = D / 32;
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int bs_mask = (1 << p.bs_log2) - 1;
    const int last = w.L - 1;
    // K: lane (n, g) loads cells tile + 8*(n/4) + 4h + (n%4), dims 32ks + 8g .. +8
    {
        const int grp = tile + 8 * (n >> 2);
        const int blk = phys_block(p, s, min(grp, last) >> p.bs_log2);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = min(grp + 4 * h + (n & 3), last);
            const int64_t row = ((int64_t) blk << p.bs_log2) | (c & bs_mask);
            const char *base = p.k_pool + row * p.k_row + (int64_t) hk * D * 2 + g * 16;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) r.k[h][ks] = *(const u32x4 *) (base + ks * 64);
        }
    }
    // V: lane (n, g) loads cells tile + 8g + e, dims (D/16)*n .. +D/16
    {
        const int grp = tile + 8 * g;
        const int blk = phys_block(p, s, min(grp, last) >> p.bs_log2);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int c = min(grp + e, last);
            const int64_t row = ((int64_t) blk << p.bs_log2) | (c & bs_mask);
            const uint32_t *src = (const uint32_t *) (p.v_pool + row * p.v_row + (int64_t) hk * D * 2 + n * (D / 8));
            if constexpr (VW == 2) {
                const u32x2 x = *(const u32x2 *) src;
                r.v[e][0] = x[0]; r.v[e][1] = x[1];
            } else {
#pragma unroll
                for (int i = 0; i < VW; i += 4) {
                    const u32x4 x = *(const u32x4 *) (src + i);
                    r.v[e][i] = x[0]; r.v[e][i + 1] = x[1]; r.v[e][i + 2] = x[2]; r.v[e][i + 3] = x[3];
                }
            }
        }
    }
}

// Per-wave running state of the online softmax for NRT row tiles.
template <int D, int NRT>
struct DecodeState {
    static constexpr int DPL = D / 16;
    f16x8 q[NRT][D / 32];
    int prow[NRT];
    float m[NRT];          // running max of row n (log2 units)
    float l[NRT];          // partial sum over this lane's cells
    f32x4 o[NRT][DPL];     // O rows 4g+i, dims DPL*n + m
};

template <int D, int NRT>
__device__ __forceinline__ void compute_tile_f16(const AttnParams &p, const SeqWindow &w, int tile,
                                                 const TileRegs<D, KV_F16> &r, DecodeState<D, NRT> &st) {
    constexpr int KS = D / 32;
    constexpr int DPL = D / 16;
    const int lane = threadIdx.x & 63, g = lane >> 4;
    // V^T B operands: MFMA m takes dim DPL*n + m of cells 8g .. 8g+7
    u32x4 vb[DPL];
#pragma unroll
    for (int m = 0; m < DPL; m++) {
        const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int wi = 0; wi < 4; wi++) vb[m][wi] = __builtin_amdgcn_perm(r.v[2 * wi + 1][m >> 1], r.v[2 * wi][m >> 1], sel);
    }
    const bool full = tile + kTile <= w.L && (!p.causal || tile + kTile - 1 <= w.pmin) &&
                      (p.n_swa <= 0 || w.pmax - tile < p.n_swa);
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        float sv[8];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, r.k[h][ks]), st.q[rt][ks], acc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) sv[4 * h + i] = acc[i];
        }
        if (p.softcap > 0.f) {
#pragma unroll
            for (int e = 0; e < 8; e++) sv[e] = p.softcap * tanhf(sv[e] * p.softcap_inv) * kLog2e;
        }
        if (!full) {
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (cell_masked(tile + 8 * g + e, w.L, st.prow[rt], p.causal, p.n_swa)) sv[e] = -INFINITY;
        }
        float mt = sv[0];
#pragma unroll
        for (int e = 1; e < 8; e++) mt = fmaxf(mt, sv[e]);
        mt = wave_max(mt);
        const float mnew = fmaxf(st.m[rt], mt);
        float alpha = 1.f;
        float pv[8];
        if (mnew == -INFINITY) {
#pragma unroll
            for (int e = 0; e < 8; e++) pv[e] = 0.f;
        } else {
            alpha = __builtin_amdgcn_exp2f(st.m[rt] - mnew);
#pragma unroll
            for (int e = 0; e < 8; e++) pv[e] = __builtin_amdgcn_exp2f(sv[e] - mnew);
        }
        st.m[rt] = mnew;
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) ps += pv[e];
        st.l[rt] = st.l[rt] * alpha + ps;
        // rescale O rows 4g+i by their row's alpha (held by lane 4g+i)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float a = __shfl(alpha, 4 * g + i);
#pragma unroll
            for (int m = 0; m < DPL; m++) st.o[rt][m][i] *= a;
        }
        u32x4 pa;
#pragma unroll
        for (int wi = 0; wi < 4; wi++) pa[wi] = pack_f16x2(pv[2 * wi], pv[2 * wi + 1]);
        const f16x8 pah = __builtin_bit_cast(f16x8, pa);
#pragma unroll
        for (int m = 0; m < DPL; m++)
            st.o[rt][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, __builtin_bit_cast(f16x8, vb[m]), st.o[rt][m], 0, 0, 0);
    }
}

template <int D, int NRT>
__global__ __launch_bounds__(64) void pa_decode_f16_kernel(AttnParams p) {
    constexpr int KS = D / 32;
    constexpr int DPL = D / 16;
    const int split = blockIdx.x, hk = blockIdx.y, s = blockIdx.z;
    const int lane = threadIdx.x, g = lane >> 4, n = lane & 15;
    SeqWindow w;
    seq_window(p, s, w);
    const int M = w.nq * p.gqa;
    if (w.nq <= 0 || M > p.decode_rows || split >= w.nsplit) return;

    DecodeState<D, NRT> st;
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        const int r = rt * 16 + n;
        st.prow[rt] = w.pmax;
        if (r < M) {
            const int t = w.q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
            st.prow[rt] = p.pos[t];
            const float *qp = p.q + ((int64_t) t * p.H + h) * D + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const float4 a = *(const float4 *) (qp + 32 * ks);
                const float4 b = *(const float4 *) (qp + 32 * ks + 4);
                const u32x4 u = {pack_f16x2(a.x * p.qscale, a.y * p.qscale), pack_f16x2(a.z * p.qscale, a.w * p.qscale),
                                 pack_f16x2(b.x * p.qscale, b.y * p.qscale), pack_f16x2(b.z * p.qscale, b.w * p.qscale)};
                st.q[rt][ks] = __builtin_bit_cast(f16x8, u);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) st.q[rt][ks] = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
        }
        st.m[rt] = -INFINITY;
        st.l[rt] = 0.f;
#pragma unroll
        for (int m = 0; m < DPL; m++) st.o[rt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int cb = w.c_lo + split * w.chunk;
    const int ce = min(w.c_hi, cb + w.chunk);
    if (cb < ce) {
        TileRegs<D, KV_F16> ra, rb;
        int tile = cb;
        load_tile_f16<D>(p, w, s, hk, tile, ra);
        while (true) {
            if (tile + kTile < ce) load_tile_f16<D>(p, w, s, hk, tile + kTile, rb);
            compute_tile_f16<D, NRT>(p, w, tile, ra, st);
            tile += kTile;
            if (tile >= ce) break;
            if (tile + kTile < ce) load_tile_f16<D>(p, w, s, hk, tile + kTile, ra);
            compute_tile_f16<D, NRT>(p, w, tile, rb, st);
            tile += kTile;
            if (tile >= ce) break;
        }
    }

#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        float l = st.l[rt];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if (w.nsplit == 1) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = rt * 16 + 4 * g + i;
                const float lr = __shfl(l, 4 * g + i);
                if (r < M) {
                    const int t = w.q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
                    const float inv = lr > 0.f ? 1.f / lr : 0.f;
                    float *op = p.out + ((int64_t) t * p.H + h) * D + DPL * n;
#pragma unroll
                    for (int m = 0; m < DPL; m += 4)
                        *(float4 *) (op + m) = make_float4(st.o[rt][m][i] * inv, st.o[rt][m + 1][i] * inv,
                                                           st.o[rt][m + 2][i] * inv, st.o[rt][m + 3][i] * inv);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = rt * 16 + 4 * g + i;
                if (r < M) {
                    const int t = w.q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
                    float *op = p.part_o + (((int64_t) t * p.H + h) * p.max_splits + split) * D + DPL * n;
#pragma unroll
                    for (int m = 0; m < DPL; m += 4)
                        *(float4 *) (op + m) = make_float4(st.o[rt][m][i], st.o[rt][m + 1][i], st.o[rt][m + 2][i], st.o[rt][m + 3][i]);
                }
            }
            const int r = rt * 16 + n;
            if (g == 0 && r < M) {
                const int t = w.q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
                float *mp = p.part_ml + (((int64_t) t * p.H + h) * p.max_splits + split) * 2;
                *(float2 *) mp = make_float2(st.m[rt], l);
            }
        }
    }
}

// Log-sum-exp merge of the split-K partials: one wave per (sequence, kv head).
template <int D>
__global__ __launch_bounds__(64) void pa_merge_kernel(AttnParams p) {
    constexpr int DL = D / 64;   // dims per lane
    const int hk = blockIdx.y, s = blockIdx.z;
    const int lane = threadIdx.x;
    SeqWindow w;
    seq_window(p, s, w);
    const int M = w.nq * p.gqa;
    if (w.nq <= 0 || M > p.decode_rows || w.nsplit == 1) return;
    for (int r = 0; r < M; r++) {
        const int t = w.q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
        const int64_t base = ((int64_t) t * p.H + h) * p.max_splits;
        float mx = -INFINITY;
        for (int sp = 0; sp < w.nsplit; sp++) mx = fmaxf(mx, p.part_ml[(base + sp) * 2]);
        float acc[DL];
#pragma unroll
        for (int i = 0; i < DL; i++) acc[i] = 0.f;
        float lsum = 0.f;
        if (mx != -INFINITY) {
            for (int sp = 0; sp < w.nsplit; sp++) {
                const float2 ml = *(const float2 *) (p.part_ml + (base + sp) * 2);
                const float wgt = __builtin_amdgcn_exp2f(ml.x - mx);   // 0 for an empty split
                lsum += wgt * ml.y;
                const float *op = p.part_o + (base + sp) * D + lane * DL;
#pragma unroll
                for (int i = 0; i < DL; i++) acc[i] += wgt * op[i];
            }
        }
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        float *out = p.out + ((int64_t) t * p.H + h) * D + lane * DL;
#pragma unroll
        for (int i = 0; i < DL; i++) out[i] = acc[i] * inv;
    }
}

template <int D, int NRT>
static hipError_t launch_decode_t(const AttnParams &p, hipStream_t stream) {
    dim3 grid(p.max_splits, p.Hkv, p.S);
    hipLaunchKernelGGL((pa_decode_f16_kernel<D, NRT>), grid, dim3(64), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.max_splits > 1) {
        hipLaunchKernelGGL((pa_merge_kernel<D>), dim3(1, p.Hkv, p.S), dim3(64), 0, stream, p);
        e = hipGetLastError();
    }
    return e;
}

hipError_t launch_decode(const AttnParams &p, int head_dim, int kv_type, hipStream_t stream) {
    if (kv_type != KV_F16) return hipErrorInvalidValue;
    const int nrt = p.decode_rows > 16 ? 2 : 1;
    switch (head_dim) {
        case 64: return nrt == 1 ? launch_decode_t<64, 1>(p, stream) : launch_decode_t<64, 2>(p, stream);
        case 128: return nrt == 1 ? launch_decode_t<128, 1>(p, stream) : launch_decode_t<128, 2>(p, stream);
        case 256: return nrt == 1 ? launch_decode_t<256, 1>(p, stream) : launch_decode_t<256, 2>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iian_pa

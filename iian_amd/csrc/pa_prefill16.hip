// pa_prefill16.hip - chunked-prefill paged attention for gfx950 with 16-row MFMA
// tiles (v_mfma_f32_16x16x32_f16), used at head size 256.
//
// At D = 256 the f16 hi/lo q pair and O of a 32-row wave take 256 registers
// alone, which leaves the 32x32 kernel (pa_prefill.hip) one wave per SIMD.
// 16-row waves keep two per SIMD; the 16x16x32 MFMA costs the same busy
// cycles per flop as the 32x32x16 form (measured on MI355X).
//
// One workgroup of NW waves per (row block, kv head, sequence); rows are
// r = j*gqa + g (query token j, head g of the GQA group), NRT 16-row MFMA tiles
// per wave.  The workgroup streams the sequence's cells in 32-cell tiles
// through the block table into LDS (register-staged double buffer) and every
// wave reuses each tile for all its rows:
//
//   S^T = K * Q^T       v_mfma_f32_16x16x32_f16, K rows read from LDS with
//                       ds_read_b128 as the A operand, Q^T from registers
//   online softmax      exp2 domain; causal / sliding-window masks only on
//                       tiles that straddle a boundary; waves skip tiles that
//                       are fully masked for all their rows
//   O += P * V          P from registers (A operand); V^T B operands come
//                       straight from the row-major LDS tile through the
//                       gfx950 transpose read ds_read_b64_tr_b16
//
// Workgroups of one (kv head, sequence) share their K/V and are placed on one
// XCD (its L2) by remapping the linear workgroup id.
// Semantics: paged_attn_impl (src/iian/paged_attn.cpp:90-146).
#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"

namespace iian_pa {

// The lo product of q in bf8 (f16 pools; pa_mfma.h): one
// v_mfma_scale_f32_16x16x128_f8f6f4 per 4 k-steps, at twice the issue time of
// one v_mfma_f32_16x16x32_f16.  Lane (n, g) byte 8j + e of block b carries
// dim 32(4b + j) + 8g + e on both sides.
__device__ __forceinline__ f32x4 mfma16_bf8_lo(const i32x8 &a, const i32x8 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 1, 1, 0, 127, 0, 127 - kLo8Shift);
}

template <int D>
struct PrefillShape16 {
    static constexpr int KS = D / 32;                 // QK^T k-steps
    static constexpr int NPV = D / 16;                // PV MFMAs (16 output dims each)
    // Padded LDS rows, both tiles stored in the order their readers walk the
    // cells: LDS row 16h + 4j + i holds cell 8j + 4h + i.  The QK^T A operand
    // (half h) then reads 16 consecutive K rows, each 4 banks after the last,
    // and a V transpose read (cells 8g + i, then 8g + 4 + i) reads rows 4g + i
    // (resp. 16 + 4g + i), 32 bytes each, 8 banks apart.
    static constexpr int KSTRIDE = D * 2 + 16;
    static constexpr int VSTRIDE = D * 2 + 32;
    static constexpr int TILE_BYTES = kTile * VSTRIDE;
    static constexpr int CHUNKS = kTile * (D / 8);    // 16-byte chunks per tile per tensor
};

typedef __attribute__((address_space(3))) s16x4 lds_s16x4_16;

__device__ __forceinline__ f16x8 lds_tr_b16x8_16(const char *p0, const char *p1) {
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_16 *) (uintptr_t) p0);
    const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_16 *) (uintptr_t) p1);
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 c = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(f16x8, c);
}

// KVT: pool type, 1 = f16, 8 = ggml Q8_0 (ggml-common.h:251-256).  A Q8_0 tile
// is staged with one thread per (tensor, cell, block): K as its exact int8
// values in f16 plus the block scales d as f32 in LDS, applied per cell after
// each QK^T k-step MFMA (k-step = block), so q*d enters the scores exactly;
// V as f16(q*d), the correctly rounded dequantised value.
template <int D, int NRT, int NW, int KVT>
// Waves per SIMD asked of the register allocator: four for f16 at D = 128 (two
// 8-wave workgroups per CU in 128 VGPRs), else two up to D = 128, one at 256.
__global__ __launch_bounds__(NW * 64, (D == 128 && KVT == 1) ? 4 : (D <= 128 ? 2 : 1)) void pa_prefill16_kernel(
    AttnParams p, int n_rb) {
    using SH = PrefillShape16<D>;
    constexpr int KS = SH::KS, NPV = SH::NPV, KSTRIDE = SH::KSTRIDE, VSTRIDE = SH::VSTRIDE;
    constexpr bool Q8 = KVT == 8;
    constexpr bool LO8 = !Q8 && KS % 4 == 0;      // lo product of q in bf8
    constexpr int CPT = SH::CHUNKS / (NW * 64);   // f16: 16-byte chunks per thread per tensor
    static_assert(Q8 || CPT * NW * 64 == SH::CHUNKS, "tile chunks must divide evenly");
    constexpr int NB = D / 32;                    // Q8_0 blocks per head slice
    constexpr int ITEMS = 2 * kTile * NB;         // Q8_0: (tensor, cell, block) staging items
    static_assert(!Q8 || ITEMS <= NW * 64, "one Q8_0 staging item per thread");
    constexpr int ROWS = NW * NRT * 16;
    __shared__ __attribute__((aligned(16))) char lds[2][2][SH::TILE_BYTES];
    __shared__ __attribute__((aligned(16))) float ksc[2][Q8 ? NB : 1][kTile];   // Q8_0 K scales [block][cell]

    // XCD-aware mapping: workgroups are dispatched round-robin over the 8 XCDs
    // (bid % 8).  (sequence, kv head) pairs are dealt round-robin to XCDs and
    // all row blocks of a pair run on its XCD, so they share K/V through that
    // XCD's L2, while neighbouring pairs (the ones that carry work when only a
    // few sequences of a batch are prefill chunks) land on different XCDs.
    const int bid = blockIdx.x;
    const int slot = bid >> 3;
    const int pair = (bid & 7) + 8 * (slot / n_rb);
    const int rb = slot % n_rb;
    if (pair >= p.S * p.Hkv) return;

    // wave index in a scalar register, so that the tile-load rows derived from
    // it stay in SALU (cfg5 global prefill 4947-5022 against 5015-5085 us)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 4,
              n = lane & 15;
    // Longest first: a workgroup holds its CU alone and the later ones take
    // the CUs that finish first, so without a sliding window the pairs are
    // dealt in decreasing order of their sequence's length (decode sequences
    // last): Gemma3-12B global-layer prefill 4146-4159 against 4958-4970 us.
    // Every workgroup ranks the batch's sequences itself, one per lane (up to
    // 64 sequences; past that, and with a window, which bounds every row
    // block's cells, the batch order stands: the ranking's round trip and
    // shuffles cost the window-bounded prefill 2-3%).
    const int hk = pair % p.Hkv;
    int s = pair / p.Hkv, L, q0, nq;
    if (p.S <= 64 && p.n_swa <= 0) {
        int ll = 0, a = 0, nql = 0, key = -1;
        if (lane < p.S) {
            ll = p.seq_lens[lane];
            a = min(max(p.qsl[lane], 0), p.T);
            nql = min(max(p.qsl[lane + 1], a), p.T) - a;
            if (nql * p.gqa > p.decode_rows) key = max(ll, 0);
        }
        int rank = 0;
        for (int j = 0; j < p.S; j++) {
            const int kj = __builtin_amdgcn_readlane(key, j);
            rank += (kj > key || (kj == key && j < lane)) ? 1 : 0;
        }
        const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < p.S && rank == s);
        s = __builtin_amdgcn_readfirstlane(hit ? (int) __builtin_ctzll(hit) : s);
        L = __builtin_amdgcn_readfirstlane(__shfl(ll, s));
        q0 = __builtin_amdgcn_readfirstlane(__shfl(a, s));
        nq = __builtin_amdgcn_readfirstlane(__shfl(nql, s));
    } else {
        L = p.seq_lens[s];
        q0 = min(max(p.qsl[s], 0), p.T);
        nq = min(max(p.qsl[s + 1], q0), p.T) - q0;
    }
    const int M = nq * p.gqa;
    // more query tokens than the caller's max_query_len: rows past this
    // launch's row blocks stay unwritten, so flag it (bit 2)
    if (rb == 0 && hk == 0 && tid == 0 && nq > p.max_q && p.err) atomicOr(p.err, 4);
    if (M <= p.decode_rows) return;
    const int R0 = rb * ROWS;
    if (R0 >= M) return;

    // positions of this workgroup's and this wave's rows
    const int Rw = R0 + wave * NRT * 16;
    int wg_min = INT32_MAX, wg_max = INT32_MIN, w_min = INT32_MAX, w_max = INT32_MIN;
    {
        const int j0 = R0 / p.gqa, j1 = (min(M, R0 + ROWS) - 1) / p.gqa;
        for (int j = j0 + lane; j <= j1; j += 64) {
            const int ps = p.pos[q0 + j];
            wg_min = min(wg_min, ps);
            wg_max = max(wg_max, ps);
        }
        if (Rw < M) {
            const int k0 = Rw / p.gqa, k1 = (min(M, Rw + NRT * 16) - 1) / p.gqa;
            for (int j = k0 + lane; j <= k1; j += 64) {
                const int ps = p.pos[q0 + j];
                w_min = min(w_min, ps);
                w_max = max(w_max, ps);
            }
        }
        for (int o = 32; o >= 1; o >>= 1) {
            wg_min = min(wg_min, __shfl_xor(wg_min, o));
            wg_max = max(wg_max, __shfl_xor(wg_max, o));
            w_min = min(w_min, __shfl_xor(w_min, o));
            w_max = max(w_max, __shfl_xor(w_max, o));
        }
    }
    const bool wave_live = Rw < M;
    int c_hi = L;
    if (p.causal) c_hi = min(c_hi, wg_max + 1);
    int c_lo = 0;
    if (p.n_swa > 0) c_lo = max(0, wg_min - p.n_swa + 1);
    c_lo &= ~(kTile - 1);

    // Q^T B operands (pre-scaled f16 hi/lo pairs; measured: +4-6% time, the
    // score error of a single f16 q removed), row positions, running state
    // (LO8: the lo half as bf8 operands, byte 8(ks%4) + e of ql8[rt][ks/4]
    // holding dim 32ks + 8g + e)
    f16x8 qv[NRT][KS], ql[NRT][LO8 ? 1 : KS];
    i32x8 ql8[NRT][LO8 ? KS / 4 : 1];
    int prow[NRT];
    float m_run[NRT], l_run[NRT];
    f32x4 o[NRT][NPV];
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        const int r = Rw + rt * 16 + n;
        prow[rt] = wave_live ? w_max : 0;
        if (r < M) {
            const int t = q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
            prow[rt] = p.pos[t];
            const float *qp = p.q + ((int64_t) t * p.H + h) * D + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                if constexpr (LO8) {
                    const float4 xa = *(const float4 *) (qp + 32 * ks), xb = *(const float4 *) (qp + 32 * ks + 4);
                    const float x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                    uint32_t w2[2] = {0u, 0u};
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float xs = x[e] * p.qscale;
                        float hv = (float) (_Float16) xs;
                        asm volatile("" : "+v"(hv));
                        qv[rt][ks][e] = (_Float16) hv;
                        w2[e >> 2] |= bf8_rne((xs - hv) * (float) (1 << kLo8Shift)) << (8 * (e & 3));
                    }
                    ql8[rt][ks / 4][2 * (ks % 4)] = (int) w2[0];
                    ql8[rt][ks / 4][2 * (ks % 4) + 1] = (int) w2[1];
                } else {
                    split_f16x8(*(const float4 *) (qp + 32 * ks), *(const float4 *) (qp + 32 * ks + 4), p.qscale,
                                qv[rt][ks], ql[rt][ks]);
                }
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) qv[rt][ks] = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int ks = 0; ks < (LO8 ? 1 : KS); ks++) ql[rt][ks] = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
            for (int b = 0; b < (LO8 ? KS / 4 : 1); b++) ql8[rt][b] = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        m_run[rt] = -INFINITY;
        l_run[rt] = 0.f;
#pragma unroll
        for (int m = 0; m < NPV; m++) o[rt][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int bs_mask = (1 << p.bs_log2) - 1;
    const int64_t head_off = (int64_t) hk * D * 2;
    // block-table entries of 64 logical blocks, one per lane, handed out with
    // lane shuffles: a tile's loads never wait on a table read
    TableWindow tw;
    if (c_lo < c_hi) table_load(p, s, c_lo >> p.bs_log2, L, tw);
    u32x4 kst[Q8 ? 1 : CPT], vst[Q8 ? 1 : CPT];
    // Q8_0 item of this thread: tensor (0 = K), cell and block; its 34 bytes
    // sit 2 bytes into (odd block) or at the start of (even block) an aligned
    // 9-dword window that stays inside the head slice
    const int qi_t = tid / (kTile * NB), qi_cell = (tid % (kTile * NB)) / NB, qi_b = tid % NB;
    const bool qi_live = Q8 && tid < ITEMS;
    uint32_t qraw[9];
    auto load_global = [&](int tile) {
        if (((min(tile + kTile - 1, L - 1) >> p.bs_log2) - tw.first) >= 64) table_load(p, s, tile >> p.bs_log2, L, tw);
        if constexpr (Q8) {
            const int c = min(tile + qi_cell, L - 1);
            const int32_t blk = __shfl(tw.id, (c >> p.bs_log2) - tw.first);
            const uint32_t row = ((uint32_t) blk << p.bs_log2) | (uint32_t) (c & bs_mask);
            if (qi_live) {
                const int start = hk * NB * 34 + 34 * qi_b;
                const uint32_t *src = (const uint32_t *) ((qi_t ? p.v_pool : p.k_pool) + pool_off(row, p.k_row) +
                                                          (start & ~3));
#pragma unroll
                for (int i = 0; i < 9; i++) qraw[i] = src[i];
            }
        } else {
#pragma unroll
            for (int j = 0; j < CPT; j++) {
                const int q = tid + j * NW * 64;
                const int cell = q / (D / 8), col = q % (D / 8);
                const int c = min(tile + cell, L - 1);
                const int32_t blk = __shfl(tw.id, (c >> p.bs_log2) - tw.first);
                const uint32_t row = ((uint32_t) blk << p.bs_log2) | (uint32_t) (c & bs_mask);
                const uint64_t off = pool_off(row, p.k_row) + (uint32_t) (head_off + col * 16);
                kst[j] = *(const u32x4 *) (p.k_pool + off);
                vst[j] = *(const u32x4 *) (p.v_pool + off);
            }
        }
    };
    auto store_lds = [&](int buf) {
        if constexpr (Q8) {
            if (!qi_live) return;
            const int lrow = ((qi_cell >> 2) & 1) * 16 + (qi_cell >> 3) * 4 + (qi_cell & 3);
            const bool odd = qi_b & 1;   // block starts 2 bytes into the window
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) (odd ? qraw[0] >> 16 : qraw[0]));
            typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
            const f16x2_t d2 = {d, d};
            u32x4 h[4];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t q4 = odd ? qraw[k + 1] : __builtin_amdgcn_alignbyte(qraw[k + 1], qraw[k], 2);
                uint32_t lo, hi;
                i8x4_to_f16(q4, lo, hi);
                if (qi_t) {   // V: f16(q*d)
                    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, lo) * d2);
                    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, hi) * d2);
                }
                h[k >> 1][2 * (k & 1)] = lo;
                h[k >> 1][2 * (k & 1) + 1] = hi;
            }
            char *dst = qi_t ? &lds[buf][1][lrow * VSTRIDE + qi_b * 64] : &lds[buf][0][lrow * KSTRIDE + qi_b * 64];
#pragma unroll
            for (int k = 0; k < 4; k++) *(u32x4 *) (dst + 16 * k) = h[k];
            if (!qi_t) ksc[buf][qi_b][qi_cell] = (float) d;
        } else {
#pragma unroll
            for (int j = 0; j < CPT; j++) {
                const int q = tid + j * NW * 64;
                const int cell = q / (D / 8), col = q % (D / 8);
                const int lrow = ((cell >> 2) & 1) * 16 + (cell >> 3) * 4 + (cell & 3);
                *(u32x4 *) (&lds[buf][0][lrow * KSTRIDE + col * 16]) = kst[j];
                *(u32x4 *) (&lds[buf][1][lrow * VSTRIDE + col * 16]) = vst[j];
            }
        }
    };

    auto compute = [&](int tile, int buf) {
        if (!wave_live) return;
        if (p.causal && tile > w_max) return;                              // every cell after every row
        if (p.n_swa > 0 && tile + kTile - 1 <= w_min - p.n_swa) return;   // every cell out of every window
        const bool full = tile + kTile <= L && (!p.causal || tile + kTile - 1 <= w_min) &&
                          (p.n_swa <= 0 || w_max - tile < p.n_swa);
        const char *Kl = lds[buf][0];
        const char *Vl = lds[buf][1];
        f16x8 ka[2][KS];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            // A operand row n of half h = cell 8(n/4) + 4h + n%4 = LDS row 16h + n
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                ka[h][ks] = *(const f16x8 *) (Kl + (16 * h + n) * KSTRIDE + (32 * ks + 8 * g) * 2);
        }
        f16x8 pa[NRT];
#pragma unroll
        for (int rt = 0; rt < NRT; rt++) {
            float sv[8];
            // issue priority up for the MFMA clusters, so that the other wave
            // on the SIMD runs its softmax in their shadow
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                if constexpr (LO8) {
#pragma unroll
                    for (int b = 0; b < KS / 4; b++) {
                        i32x8 a8;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int ks = 4 * b + j;
                            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[h][ks], qv[rt][ks], acc, 0, 0, 0);
                            const u32x4 au = __builtin_bit_cast(u32x4, ka[h][ks]);
                            a8[2 * j] = (int) f16x4_top_bytes(au[0], au[1]);
                            a8[2 * j + 1] = (int) f16x4_top_bytes(au[2], au[3]);
                        }
                        acc = mfma16_bf8_lo(a8, ql8[rt][b], acc);
                    }
                }
#pragma unroll
                for (int ks = 0; ks < (LO8 ? 0 : KS); ks++) {
                    if constexpr (Q8) {
                        // this lane's S^T rows are cells 8g + 4h + i; k-step ks = Q8_0 block ks
                        f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[h][ks], qv[rt][ks],
                                                                         f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[h][ks], ql[rt][ks], c, 0, 0, 0);
                        const f32x4 dk = *(const f32x4 *) &ksc[buf][ks][8 * g + 4 * h];
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[i] = fmaf(c[i], dk[i], acc[i]);
                    } else {
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[h][ks], qv[rt][ks], acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[h][ks], ql[rt][ks], acc, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; i++) sv[4 * h + i] = acc[i];
            }
            __builtin_amdgcn_s_setprio(0);
            if (p.softcap > 0.f) {
#pragma unroll
                for (int e = 0; e < 8; e++) sv[e] = p.softcap * tanhf(sv[e] * p.softcap_inv) * kLog2e;
            }
            if (!full) {
                const CellWindow cw = cell_window(tile + 8 * g, 8, L, prow[rt], p.causal, p.n_swa);
#pragma unroll
                for (int e = 0; e < 8; e++) sv[e] = cell_visible(cw, e) ? sv[e] : -INFINITY;
            }
            // Lazy rescale: the row's reference max m_run moves only when a
            // score exceeds it by more than kRescaleSlack; the test is on the
            // lane's own 8 cells, and the row-wide max is formed only on the
            // (rare, wave-uniform) tiles where some lane trips it.
            float lmax = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                               fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
            if (__builtin_amdgcn_ballot_w64(lmax > m_run[rt] + kRescaleSlack)) {
                const float mt = wave_max(lmax);
                const bool grow = mt > m_run[rt] + kRescaleSlack;
                const float mnew = grow ? mt : m_run[rt];
                const float alpha = grow ? __builtin_amdgcn_exp2f(m_run[rt] - mnew) : 1.f;   // 0 from -inf
                m_run[rt] = mnew;
                l_run[rt] *= alpha;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float a = __shfl(alpha, 4 * g + i);   // alpha of O row 4g+i
#pragma unroll
                    for (int m = 0; m < NPV; m++) o[rt][m][i] *= a;
                }
            }
            // a row with m_run = -inf has only masked cells so far: its P is 0
            const float mref = m_run[rt] == -INFINITY ? 0.f : m_run[rt];
            // The row sum accumulates the f16 P the PV MFMA consumes (lane-partial;
            // reduced over the lane groups at the end).  Each f16 pair is its own
            // value: hipcc (ROCm 7.2) fed v_dot2c the first dword four times when
            // the pairs were taken as elements of the packed u32x4.
            typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
            const f16x2v one2 = {(_Float16) 1.0f, (_Float16) 1.0f};
            u32x4 pk;
#pragma unroll
            for (int wi = 0; wi < 4; wi++) {
                const f16x2v h2 = {(_Float16) __builtin_amdgcn_exp2f(sv[2 * wi] - mref),
                                   (_Float16) __builtin_amdgcn_exp2f(sv[2 * wi + 1] - mref)};
                l_run[rt] = __builtin_amdgcn_fdot2(h2, one2, l_run[rt], false);
                pk[wi] = __builtin_bit_cast(uint32_t, h2);
            }
            pa[rt] = __builtin_bit_cast(f16x8, pk);
        }
        const char *vrow = Vl + (4 * g + (n >> 2)) * VSTRIDE + 8 * (n & 3);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int m = 0; m < NPV; m++) {
            const f16x8 vb = lds_tr_b16x8_16(vrow + 32 * m, vrow + 16 * VSTRIDE + 32 * m);
#pragma unroll
            for (int rt = 0; rt < NRT; rt++) o[rt][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[rt], vb, o[rt][m], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    };

    if (c_lo < c_hi) {
        int buf = 0;
        load_global(c_lo);
        store_lds(0);
        __syncthreads();
        for (int tile = c_lo; tile < c_hi; tile += kTile) {
            const bool has_next = tile + kTile < c_hi;
            if (has_next) load_global(tile + kTile);
            compute(tile, buf);
            if (has_next) store_lds(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    }

    if (!wave_live) return;
#pragma unroll
    for (int rt = 0; rt < NRT; rt++) {
        float l = l_run[rt];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = Rw + rt * 16 + 4 * g + i;
            const float lr = __shfl(l, 4 * g + i);
            if (r < M) {
                const int t = q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
                const float inv = lr > 0.f ? 1.f / lr : 0.f;
                float *op = p.out + ((int64_t) t * p.H + h) * D + n;
#pragma unroll
                for (int m = 0; m < NPV; m++) op[16 * m] = o[rt][m][i] * inv;
            }
        }
    }
}

template <int D, int NRT, int NW, int KVT>
static hipError_t launch_prefill16_t(const AttnParams &p, int max_rows, hipStream_t stream) {
    constexpr int ROWS = NW * NRT * 16;
    const int n_rb = (max_rows + ROWS - 1) / ROWS;
    const int pairs_per_xcd = (p.S * p.Hkv + 7) / 8;
    const int nwg = 8 * pairs_per_xcd * n_rb;
    hipLaunchKernelGGL((pa_prefill16_kernel<D, NRT, NW, KVT>), dim3(nwg), dim3(NW * 64), 0, stream, p, n_rb);
    return hipGetLastError();
}

hipError_t launch_prefill16(const AttnParams &p, int head_dim, int kv_type, int max_rows, hipStream_t stream) {
    if (head_dim != 256) return hipErrorInvalidValue;
    switch (kv_type) {
        case 1: return launch_prefill16_t<256, 1, 8, 1>(p, max_rows, stream);
        case 8: return launch_prefill16_t<256, 1, 8, 8>(p, max_rows, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iian_pa

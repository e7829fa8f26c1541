// pa_prefill.hip - chunked-prefill causal paged attention for gfx950 (MFMA 32x32x16 f16, LDS-staged KV).
//
// One workgroup of NW waves per (row block, kv head, sequence); rows are
// r = j*gqa + g (query token j, head g of the GQA group) and every wave owns 32
// of them.  The workgroup streams the sequence's cells in 64-cell tiles
// through the block table into a double-buffered LDS tile pair and every wave
// reuses each tile for its 32 rows.  f16 tiles at D >= 128 go straight from
// HBM to LDS (global_load_lds_dwordx4, rows unpadded with their 16-byte chunks
// XOR-swizzled, issued from inline asm so that reads of the other buffer do not
// wait on them); D = 64 and 96 and Q8_0 tiles are staged through registers
// (padded rows).  Per tile:
//
//   S^T = K * Q^T       v_mfma_f32_32x32x16_f16: K rows (cells) from LDS with
//                       ds_read_b128 as the A operand, Q^T (f16 hi/lo pair)
//                       from registers as the B operand; the tile's two
//                       32-cell halves are two independent accumulation chains
//   online softmax      exp2 domain; lane l holds 32 cells of query row l%32,
//                       lane l^32 the other 32; causal / sliding-window masks
//                       only on tiles that straddle a boundary; waves skip
//                       tiles that are fully masked for all their rows
//   O += P * V          P straight from the S^T registers as the A operand (the
//                       k positions of a PV step are the cells the lane holds);
//                       V B operands from the row-major LDS tile through the
//                       gfx950 transpose read ds_read_b64_tr_b16
//
// 32 rows per wave halve the LDS bytes read per flop against 16-row tiles.
// A chain of dependent MFMAs issues at ~64% of the MFMA rate on MI355X
// (measured: one 32x32x16 accumulator per wave 1.58 PFLOP/s, two 2.11, four
// 2.44), so a tile carries two independent S^T chains and PV four output tiles.
//
// MFMA 32x32x16 operand layouts (lane l, h = l/32): A[m][k] holds
// A[l%32][8h .. 8h+7]; B holds B[8h .. 8h+7][l%32]; the f32 result register r
// holds D[8(r/4) + 4h + r%4][l%32].
//
// Workgroups of one (kv head, sequence) share their K/V and are placed on one
// XCD (its L2) by remapping the linear workgroup id.
// Semantics: paged_attn_impl (src/iian/paged_attn.cpp:90-146).
#include "pa_common.h"
#include "pa_launch.h"
#include "pa_mfma.h"
#include "pa_decode_body.h"

#ifndef IIAN_PA_PREFILL_LO8
#define IIAN_PA_PREFILL_LO8 1
#endif

namespace iian_pa {

// Waves per SIMD asked of the register allocator: two at D <= 128 (two 4-wave
// workgroups per CU in 256 registers), one at D = 256 (O and the q pair take
// 256 registers alone).
template <int D>
struct PrefillOcc {
    static constexpr int kWavesPerSimd = D <= 128 ? 2 : 1;
};

// KVT: pool type, 1 = f16, 8 = ggml Q8_0 (ggml-common.h:251-256).  A Q8_0 tile
// is staged with one thread per (tensor, cell, block): K as its exact int8
// values in f16 plus the block scales d as f32 in LDS, applied per cell after
// the two QK^T k-steps of each block, so q*d enters the scores exactly; V as
// f16(q*d), the correctly rounded dequantised value.
//
// MIXED: the launch of a mixed batch over an f16 pool.  The first n_dec
// workgroups hold NW stream-K decode workers each (one wave per worker,
// decode_piece of pa_decode_body.h) and are dispatched first, on three CUs in
// four (kF16MixedDecodeWavesPerCu in pa_abi.hip): the HBM-bound decode waves
// and the MFMA-bound prefill workgroups then share those CUs from the start,
// instead of the decode rows waiting for the prefill tail.  Split decode segments are merged inside the launch (arrive_last):
// the decode workers finish long before the prefill workgroups, so the merge
// costs the launch nothing, and the call is one launch.
template <int D, int NW, int KVT, bool MIXED>
__global__ __launch_bounds__(NW * 64, PrefillOcc<D>::kWavesPerSimd) void pa_prefill_kernel(AttnParams p, int n_rb,
                                                                                          int n_dec) {
    int bid = blockIdx.x;
    if constexpr (MIXED) {
        if (bid < n_dec) {
            const int worker = bid * NW + (int) (threadIdx.x >> 6);
            if (worker < p.sk_workers)
                for_each_piece<false>(p, worker, 0,
                                      [&](const SeqWindow &w, const Piece &pc) { decode_piece<D, 1, true>(p, w, pc); });
            return;
        }
        bid -= n_dec;   // a multiple of 8: the XCD of every prefill workgroup is unchanged
    }
    constexpr bool DMA = KVT == 1 && D >= 128;   // f16 tiles loaded straight into LDS
    using SH = PrefillShape<D, DMA>;
    constexpr int KK = SH::KK, NO = SH::NO, KSTRIDE = SH::KSTRIDE, VSTRIDE = SH::VSTRIDE;
    constexpr int PT = SH::PT, NH = SH::NH, NS = 16 * NH;   // cells per tile, 32-cell halves, scores per lane
    constexpr bool Q8 = KVT == 8;
    constexpr bool LO8 = !Q8 && IIAN_PA_PREFILL_LO8;   // lo product of q in bf8 (pa_mfma.h)
    constexpr int NB8 = (KK + 3) / 4;                   // bf8 lo MFMAs per 32-cell half (the last one partial at D = 96)
    constexpr int NT = NW * 64;
    constexpr int CPT = SH::CHUNKS / NT;          // f16: 16-byte chunks per thread per tensor
    static_assert(Q8 || CPT * NT == SH::CHUNKS, "tile chunks must divide evenly");
    constexpr int NB = D / 32;                    // Q8_0 blocks per head slice
    constexpr int ITEMS = 2 * PT * NB;        // Q8_0: (tensor, cell, block) staging items
    constexpr int IPT = (ITEMS + NT - 1) / NT;    // Q8_0 items per thread
    constexpr int ROWS = NW * 32;
    // double-buffered K/V tiles
    __shared__ __attribute__((aligned(16))) char lds_k0[SH::KBYTES];
    __shared__ __attribute__((aligned(16))) char lds_k1[SH::KBYTES];
    __shared__ __attribute__((aligned(16))) char lds_v0[SH::VBYTES];
    __shared__ __attribute__((aligned(16))) char lds_v1[SH::VBYTES];
    __shared__ __attribute__((aligned(16))) float ksc[2][Q8 ? NB : 1][PT];   // Q8_0 K scales [block][cell]

    // XCD-aware mapping: workgroups are dispatched round-robin over the 8 XCDs
    // (bid % 8) and within an XCD round-robin over its CUs, so the XCD's slots
    // s and s + cus_per_xcd share a CU.  (sequence, kv head) pairs are dealt
    // round-robin to XCDs and all row blocks of a pair run on its XCD, so they
    // share K/V through that XCD's L2, while neighbouring pairs (the ones that
    // carry work when only a few sequences of a batch are prefill chunks) land
    // on different XCDs.  A pair whose first slot falls in an odd round of
    // slots takes its row blocks in reverse, so that a pair's heavy late row
    // blocks (they attend the most cells) share CUs with another pair's light
    // early ones and get the CU to themselves sooner (Qwen3-8B chunked prefill
    // 133.3-134.0 against 137.2-137.3 us; with decode rows 164.8-165.9 against
    // 173.5-173.7 us).  Per pair, so every row block is taken once.
    const int slot = bid >> 3;
    const int pair_x = slot / n_rb;
    const int pair = (bid & 7) + 8 * pair_x;
    const int rb = (((pair_x * n_rb) / p.cus_per_xcd) & 1) ? n_rb - 1 - slot % n_rb : slot % n_rb;
    if (pair >= p.S * p.Hkv) return;
    const int s = pair / p.Hkv;
    const int hk = pair % p.Hkv;

    // wave index in a scalar register: the DMA rows, block ids and LDS
    // addresses derived from it then stay in SALU (-1.5% at the Qwen3-8B
    // chunked-prefill shape, against about 11 VALU per DMA pair in VGPRs)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, hh = lane >> 5,
              n = lane & 31;
    const int L = p.seq_lens[s];
    const int q0 = min(max(p.qsl[s], 0), p.T);
    const int nq = min(max(p.qsl[s + 1], q0), p.T) - q0;
    const int M = nq * p.gqa;
    // more query tokens than the caller's max_query_len: rows past this
    // launch's row blocks stay unwritten, so flag it (bit 2)
    if (rb == 0 && hk == 0 && threadIdx.x == 0 && nq > p.max_q && p.err) atomicOr(p.err, 4);
    if (M <= p.decode_rows) return;
    const int R0 = rb * ROWS;
    if (R0 >= M) return;

    // positions of this workgroup's and this wave's rows
    const int Rw = R0 + wave * 32;
    int wg_min = INT32_MAX, wg_max = INT32_MIN, w_min = INT32_MAX, w_max = INT32_MIN;
    {
        const int j0 = R0 / p.gqa, j1 = (min(M, R0 + ROWS) - 1) / p.gqa;
        for (int j = j0 + lane; j <= j1; j += 64) {
            const int ps = p.pos[q0 + j];
            wg_min = min(wg_min, ps);
            wg_max = max(wg_max, ps);
        }
        if (Rw < M) {
            const int k0 = Rw / p.gqa, k1 = (min(M, Rw + 32) - 1) / p.gqa;
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
        // equal in every lane after the butterflies: scalars from here on
        wg_min = __builtin_amdgcn_readfirstlane(wg_min);
        wg_max = __builtin_amdgcn_readfirstlane(wg_max);
        w_min = __builtin_amdgcn_readfirstlane(w_min);
        w_max = __builtin_amdgcn_readfirstlane(w_max);
    }
    const bool wave_live = Rw < M;
    int c_hi = L;
    if (p.causal) c_hi = min(c_hi, wg_max + 1);
    int c_lo = 0;
    if (p.n_swa > 0) c_lo = max(0, wg_min - p.n_swa + 1);
    c_lo &= ~(kTile - 1);

    // Q^T B operands of query row n (pre-scaled f16 hi/lo pairs, dims
    // 16kk + 8hh .. +7), its position and running state.  The pair carries q
    // to ~2^-22 relative (split_f16x8).
    // LO8 (f16 pools): the lo half as bf8 operands of the scaled fp8 MFMA,
    // byte 8(kk%4) + e of ql8[kk/4] holding dim 16kk + 8hh + e (pa_mfma.h),
    // where the K operand bytes of the same dims sit; bytes past dim D are 0
    f16x8 qv[KK], ql[LO8 ? 1 : KK];
    i32x8 ql8[LO8 ? NB8 : 1];
#pragma unroll
    for (int b = 0; b < (LO8 ? NB8 : 1); b++) ql8[b] = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
    const int qr = Rw + n;
    int prow = wave_live ? w_max : 0;
    if (qr < M) {
        const int t = q0 + qr / p.gqa, h = hk * p.gqa + qr % p.gqa;
        prow = p.pos[t];
        const float *qp = p.q + ((int64_t) t * p.H + h) * D + 8 * hh;
#pragma unroll
        for (int kk = 0; kk < KK; kk++) {
            if constexpr (LO8) {
                const float4 xa = *(const float4 *) (qp + 16 * kk), xb = *(const float4 *) (qp + 16 * kk + 4);
                const float x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                uint32_t w2[2] = {0u, 0u};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float xs = x[e] * p.qscale;
                    float hv = (float) (_Float16) xs;
                    asm volatile("" : "+v"(hv));
                    qv[kk][e] = (_Float16) hv;
                    w2[e >> 2] |= bf8_rne((xs - hv) * (float) (1 << kLo8Shift)) << (8 * (e & 3));
                }
                ql8[kk / 4][2 * (kk % 4)] = (int) w2[0];
                ql8[kk / 4][2 * (kk % 4) + 1] = (int) w2[1];
            } else {
                split_f16x8(*(const float4 *) (qp + 16 * kk), *(const float4 *) (qp + 16 * kk + 4), p.qscale, qv[kk],
                            ql[kk]);
            }
        }
    } else {
#pragma unroll
        for (int kk = 0; kk < KK; kk++) qv[kk] = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
        for (int kk = 0; kk < (LO8 ? 1 : KK); kk++) ql[kk] = __builtin_bit_cast(f16x8, u32x4{0u, 0u, 0u, 0u});
    }
    float m_run = -INFINITY, l_run = 0.f;   // of query row n (same in lanes n and n + 32)
    f32x16 o[NO];                           // O rows 8(r/4) + 4hh + r%4, dims 32m + n
#pragma unroll
    for (int m = 0; m < NO; m++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[m][r] = 0.f;

    const int bs_mask = (1 << p.bs_log2) - 1;
    const int64_t head_off = (int64_t) hk * D * 2;
    // block-table entries of 64 logical blocks, one per lane, handed out with
    // lane shuffles: a tile's loads never wait on a table read
    TableWindow tw;
    if (c_lo < c_hi) table_load(p, s, c_lo >> p.bs_log2, L, tw);
    u32x4 kst[(Q8 || DMA) ? 1 : CPT], vst[(Q8 || DMA) ? 1 : CPT];
    // Q8_0 items of this thread: tensor (0 = K), cell and block; its 34 bytes
    // sit 2 bytes into (odd block) or at the start of (even block) an aligned
    // 9-dword window that stays inside the head slice
    uint32_t qraw[Q8 ? IPT : 1][9];
    auto load_global = [&](int tile) {
        if (((min(tile + PT - 1, L - 1) >> p.bs_log2) - tw.first) >= 64) table_load(p, s, tile >> p.bs_log2, L, tw);
        if constexpr (Q8) {
#pragma unroll
            for (int it = 0; it < IPT; it++) {
                const int item = tid + it * NT;
                const int qi_t = item / (PT * NB), qi_cell = (item % (PT * NB)) / NB, qi_b = item % NB;
                const int c = min(tile + qi_cell, L - 1);
                const int32_t blk = __shfl(tw.id, (c >> p.bs_log2) - tw.first);
                const uint32_t row = ((uint32_t) blk << p.bs_log2) | (uint32_t) (c & bs_mask);
                if (item < ITEMS) {
                    const int start = hk * NB * 34 + 34 * qi_b;
                    const uint32_t *src = (const uint32_t *) ((qi_t ? p.v_pool : p.k_pool) + pool_off(row, p.k_row) +
                                                              (start & ~3));
#pragma unroll
                    for (int i = 0; i < 9; i++) qraw[it][i] = src[i];
                }
            }
        } else if constexpr (!DMA) {
#pragma unroll
            for (int j = 0; j < CPT; j++) {
                const int q = tid + j * NT;
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
    // DMA tiles: wave instruction q of a tensor fills tile bytes [1024q, 1024q + 1024);
    // lane i's 16 bytes land at 1024q + 16i = row r, chunk slot (16i % 2D)/16,
    // which holds the row's logical chunk slot ^ swz(r)
    // Rows of a wave instruction: 1024 bytes = RI rows of 2D bytes, rows
    // RI*q .. RI*q + RI - 1 of the tile, inside one block (RI <= 8 <= block
    // size, RI*q a multiple of RI).  On a tile that ends inside the sequence
    // the block id is therefore wave-uniform (a readlane of the table window)
    // and the lane's part of the address is a per-wave constant.
    constexpr int RI = 1024 / (2 * D);
    static_assert(!DMA || (RI <= 8 && (NW * RI) % 16 == 0), "a DMA instruction's rows stay in one block");
    const int64_t dma_lane_off =
        (int64_t) (lane / (2 * D / 16)) * p.k_row + head_off +
        16 * ((lane % (2 * D / 16)) ^ swz((RI * wave + lane / (2 * D / 16)) & 15));
    const uint32_t dma_lane_off32 = (uint32_t) dma_lane_off;
    auto load_dma = [&](int tile, char *Kd, char *Vd) {
        if (((min(tile + PT - 1, L - 1) >> p.bs_log2) - tw.first) >= 64) table_load(p, s, tile >> p.bs_log2, L, tw);
        constexpr int NQ = SH::KBYTES / 1024 / NW;   // instructions per wave per tensor
        if (tile + PT <= L) {
#pragma unroll
            for (int j = 0; j < NQ; j++) {
                const int r0 = RI * (j * NW + wave);   // first row of this instruction
                const int blk = __builtin_amdgcn_readlane(tw.id, ((tile + r0) >> p.bs_log2) - tw.first);
                const uint32_t row = ((uint32_t) blk << p.bs_log2) | (uint32_t) ((tile + r0) & bs_mask);
                const uint32_t lk = __builtin_amdgcn_readfirstlane((uint32_t) (uintptr_t) (Kd + (j * NW + wave) * 1024));
                const uint32_t lv = __builtin_amdgcn_readfirstlane((uint32_t) (uintptr_t) (Vd + (j * NW + wave) * 1024));
                // the rows' base in SGPRs, the lane's part a 32-bit offset
                // (below 4 rows: the host admits rows shorter than 1 GiB)
                const uint64_t rbase = pool_off(row, p.k_row);
                lds_load16_s(p.k_pool + rbase, dma_lane_off32, lk);
                lds_load16_s(p.v_pool + rbase, dma_lane_off32, lv);
            }
            return;
        }
        // the sequence's last tile: rows past L-1 repeat cell L-1 (per lane;
        // the lane index passes through opaque() so that none of this is
        // held in registers across the tile loop)
        const int ln = (int) opaque((uint32_t) lane);
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            const int q = j * NW + wave;
            const int b = q * 1024 + 16 * ln;
            const int r = b / (2 * D), slot = (b % (2 * D)) >> 4;
            const int c = min(tile + r, L - 1);
            const int32_t blk = __shfl(tw.id, (c >> p.bs_log2) - tw.first);
            const uint32_t row = ((uint32_t) blk << p.bs_log2) | (uint32_t) (c & bs_mask);
            const uint64_t off = pool_off(row, p.k_row) + (uint32_t) (head_off + 16 * (slot ^ swz(r & 15)));
            const uint32_t lk = __builtin_amdgcn_readfirstlane((uint32_t) (uintptr_t) (Kd + q * 1024));
            const uint32_t lv = __builtin_amdgcn_readfirstlane((uint32_t) (uintptr_t) (Vd + q * 1024));
            lds_load16(p.k_pool + off, lk);
            lds_load16(p.v_pool + off, lv);
        }
    };
    auto store_lds = [&](int buf) {
        if constexpr (Q8) {
#pragma unroll
            for (int it = 0; it < IPT; it++) {
                const int item = tid + it * NT;
                if (item >= ITEMS) continue;
                const int qi_t = item / (PT * NB), qi_cell = (item % (PT * NB)) / NB, qi_b = item % NB;
                const bool odd = qi_b & 1;   // block starts 2 bytes into the window
                const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) (odd ? qraw[it][0] >> 16 : qraw[it][0]));
                typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
                const f16x2_t d2 = {d, d};
                u32x4 hv[4];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t q4 = odd ? qraw[it][k + 1] : __builtin_amdgcn_alignbyte(qraw[it][k + 1], qraw[it][k], 2);
                    uint32_t lo, hi;
                    i8x4_to_f16(q4, lo, hi);
                    if (qi_t) {   // V: f16(q*d)
                        lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, lo) * d2);
                        hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, hi) * d2);
                    }
                    hv[k >> 1][2 * (k & 1)] = lo;
                    hv[k >> 1][2 * (k & 1) + 1] = hi;
                }
                char *dst = qi_t ? (buf ? lds_v1 : lds_v0) + qi_cell * VSTRIDE + qi_b * 64
                                 : (buf ? lds_k1 : lds_k0) + qi_cell * KSTRIDE + qi_b * 64;
#pragma unroll
                for (int k = 0; k < 4; k++) *(u32x4 *) (dst + 16 * k) = hv[k];
                if (!qi_t) ksc[buf][qi_b][qi_cell] = (float) d;
            }
        } else if constexpr (!DMA) {
#pragma unroll
            for (int j = 0; j < CPT; j++) {
                const int q = tid + j * NT;
                const int cell = q / (D / 8), col = q % (D / 8);
                *(u32x4 *) ((buf ? lds_k1 : lds_k0) + cell * KSTRIDE + col * 16) = kst[j];
                *(u32x4 *) ((buf ? lds_v1 : lds_v0) + cell * VSTRIDE + col * 16) = vst[j];
            }
        }
    };

    auto compute = [&](int tile, int buf, const char *Kl, const char *Vl) {
        if (!wave_live) return;
        if (p.causal && tile > w_max) return;                               // every cell after every row
        if (p.n_swa > 0 && tile + PT - 1 <= w_min - p.n_swa) return;   // every cell out of every window
        const bool full = tile + PT <= L && (!p.causal || tile + PT - 1 <= w_min) &&
                          (p.n_swa <= 0 || w_max - tile < p.n_swa);

        // S^T = K Q^T for the tile's two 32-cell halves (independent chains;
        // the hi and lo products of a half accumulate in its chain).  Register
        // r of half c holds cell 32c + 8(r/4) + 4hh + r%4.
        // The accumulators start at -mofs, the row's reference max, so that a
        // full tile's scores come out relative to it and feed exp2 directly
        // (not with a softcap, which must see the raw score).
        const float mofs = (p.softcap > 0.f || m_run == -INFINITY) ? 0.f : m_run;
        f32x16 sa[NH];
#pragma unroll
        for (int c = 0; c < NH; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) sa[c][r] = -mofs;
        // A row = cell 32c + n, dims 16kk + 8hh (tile bytes 32kk + 16hh)
        if constexpr (Q8) {
            // k-steps 2b, 2b+1 make Q8_0 block b; its scale d_K[cell] multiplies
            // the block's partial product per S^T row
#pragma unroll
            for (int b = 0; b < NB; b++) {
                f32x16 cb[NH];
#pragma unroll
                for (int c = 0; c < NH; c++)
#pragma unroll
                    for (int r = 0; r < 16; r++) cb[c][r] = 0.f;
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int c = 0; c < NH; c++) {
                        const f16x8 a = *(const f16x8 *) (Kl + 32 * c * KSTRIDE +
                                                          tile_off<D, DMA>(n, 32 * (2 * b + u) + 16 * hh, KSTRIDE));
                        cb[c] = mfma32(a, qv[2 * b + u], cb[c]);
                        cb[c] = mfma32(a, ql[2 * b + u], cb[c]);
                    }
#pragma unroll
                for (int c = 0; c < NH; c++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const f32x4 dk = *(const f32x4 *) &ksc[buf][b][32 * c + 8 * i + 4 * hh];
#pragma unroll
                        for (int j = 0; j < 4; j++) sa[c][4 * i + j] = fmaf(cb[c][4 * i + j], dk[j], sa[c][4 * i + j]);
                    }
            }
        } else {
            // Issue priority up for the MFMA clusters (QK^T here, PV below):
            // of the two waves on a SIMD, the one with MFMAs to issue goes
            // first and the other's softmax VALU fills the MFMA shadow, instead
            // of both waves reaching their softmax at the same time (measured
            // -5% at the Qwen3-8B chunked-prefill shape).
            uint32_t ka[KK];   // this tile's read bases of k-step kk (row n of half 0)
#pragma unroll
            for (int kk = 0; kk < KK; kk++) ka[kk] = opaque(lds_addr(Kl + tile_off<D, DMA>(n, 32 * kk + 16 * hh, KSTRIDE)));
            __builtin_amdgcn_s_setprio(1);
            if constexpr (LO8) {
                // hi product per k-step in f16; the lo product per 4 k-steps
                // in bf8, its K operand the top bytes of the same f16 reads
                // K reads run AH reads ahead of their MFMA (rotating
                // registers; scheduling fences keep the compiler from sinking
                // each read next to its use, which left the read latency
                // exposed on every k-step: cfg3_prefill 135.8 against 125.9 us
                // with 4 ahead, 126.1-126.2 with 2 or 3; a workgroup alone on
                // its CU, one wave per SIMD, has no other wave to hide it)
                constexpr int NR = KK * NH, AH = 4;
                auto rd = [&](int r) { return lds_read_f16x8(ka[r / NH] + 32 * (r % NH) * KSTRIDE); };
                f16x8 ab[AH + 1];
#pragma unroll
                for (int r = 0; r < AH; r++) ab[r] = rd(r);
                i32x8 a8[NH];
#pragma unroll
                for (int r = 0; r < NR; r++) {
                    const int kk = r / NH, c = r % NH, j = kk % 4;
                    if (r + AH < NR) ab[(r + AH) % (AH + 1)] = rd(r + AH);
                    __builtin_amdgcn_sched_barrier(0);
                    const f16x8 a = ab[r % (AH + 1)];
                    sa[c] = mfma32(a, qv[kk], sa[c]);
                    const u32x4 au = __builtin_bit_cast(u32x4, a);
                    a8[c][2 * j] = (int) f16x4_top_bytes(au[0], au[1]);
                    a8[c][2 * j + 1] = (int) f16x4_top_bytes(au[2], au[3]);
                    if (kk == KK - 1 && (KK % 4) != 0) {   // D = 96: the last block's bytes past dim D are 0
#pragma unroll
                        for (int jj = KK % 4; jj < 4; jj++) a8[c][2 * jj] = a8[c][2 * jj + 1] = 0;
                    }
                    if (c == NH - 1 && (j == 3 || kk == KK - 1)) {
#pragma unroll
                        for (int cc = 0; cc < NH; cc++) sa[cc] = mfma32_bf8_lo(a8[cc], ql8[kk / 4], sa[cc]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < KK; kk++)
#pragma unroll
                    for (int c = 0; c < NH; c++) {
                        const f16x8 a = lds_read_f16x8(ka[kk] + 32 * c * KSTRIDE);
                        sa[c] = mfma32(a, qv[kk], sa[c]);
                        sa[c] = mfma32(a, ql[kk], sa[c]);
                    }
                // keep four K operand reads in flight ahead of the MFMAs instead of
                // waiting on each read right before its MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
                for (int j = 0; j < NH * KK - 4; j++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            }
            __builtin_amdgcn_s_setprio(0);
        }
        float sv[NS];   // scores relative to mofs
#pragma unroll
        for (int c = 0; c < NH; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) sv[16 * c + r] = sa[c][r];
        if (p.softcap > 0.f) {
#pragma unroll
            for (int e = 0; e < NS; e++) sv[e] = p.softcap * tanhf(sv[e] * p.softcap_inv) * kLog2e;
        }
        if (!full) {
            // score e is cell tile + 4hh + 32(e/16) + 8((e%16)/4) + e%4
            const CellWindow cw = cell_window(tile + 4 * hh, PT, L, prow, p.causal, p.n_swa);
#pragma unroll
            for (int e = 0; e < NS; e++) {
                const int r = e & 15;
                sv[e] = cell_visible(cw, 32 * (e >> 4) + 8 * (r >> 2) + (r & 3)) ? sv[e] : -INFINITY;
            }
        }
        // Lazy rescale: the row's reference max m_run moves only when a score
        // exceeds it by more than kRescaleSlack; the test is on the lane's own
        // 32 cells, and the row max is formed only on the (rare, wave-uniform)
        // tiles where some lane trips it.
        float lmax = sv[0];
#pragma unroll
        for (int e = 1; e < NS; e++) lmax = fmaxf(lmax, sv[e]);
        lmax += mofs;   // the lane's largest score
        if (__builtin_amdgcn_ballot_w64(lmax > m_run + kRescaleSlack)) {
            const float mt = fmaxf(lmax, __shfl_xor(lmax, 32));
            const bool grow = mt > m_run + kRescaleSlack;
            const float mnew = grow ? mt : m_run;
            const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - mnew) : 1.f;   // 0 from -inf
            m_run = mnew;
            l_run *= alpha;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float a = __shfl(alpha, 8 * (r >> 2) + 4 * hh + (r & 3));   // alpha of O row of register r
#pragma unroll
                for (int m = 0; m < NO; m++) o[m][r] *= a;
            }
        }
        // exp2 argument = score - m_run = sv + (mofs - m_run): no correction on
        // a tile whose accumulators started at the current reference max.  A
        // row with m_run = -inf has only masked cells so far (sv = -inf): P = 0.
        const float delta = m_run == -INFINITY ? 0.f : mofs - m_run;
        if (__builtin_amdgcn_ballot_w64(delta != 0.f)) {
#pragma unroll
            for (int e = 0; e < NS; e++) sv[e] += delta;
        }
        // The row sum accumulates the f16 P the PV MFMA consumes (lane-partial;
        // the two lane halves are added at the end).  Each f16 pair is its own
        // value: hipcc (ROCm 7.2) fed v_dot2c the first dword four times when
        // the pairs were taken as elements of a packed u32x4.
        typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
        const f16x2v one2 = {(_Float16) 1.0f, (_Float16) 1.0f};
        f16x8 pa[2 * NH];   // PV step 2c + a: registers 8a .. 8a+7 of half c = cells 32c + 16a + 4hh + {0..3, 8..11}
#pragma unroll
        for (int st = 0; st < 2 * NH; st++) {
            u32x4 pk;
#pragma unroll
            for (int wi = 0; wi < 4; wi++) {
                const f16x2v h2 = {(_Float16) __builtin_amdgcn_exp2f(sv[8 * st + 2 * wi]),
                                   (_Float16) __builtin_amdgcn_exp2f(sv[8 * st + 2 * wi + 1])};
                l_run = __builtin_amdgcn_fdot2(h2, one2, l_run, false);
                pk[wi] = __builtin_bit_cast(uint32_t, h2);
            }
            pa[st] = __builtin_bit_cast(f16x8, pk);
        }
        // V^T B operand of PV step st, output tile m: lane group l/16 reads rows
        // 16st + 4hh + i/4 (then + 8) at dims 32m + 16((l/16)%2) + 4(i%4) and
        // receives dim 32m + l%32 of the 4 cells
        const int gi = lane & 15, vr = 4 * hh + (gi >> 2), vb0 = (16 * ((lane >> 4) & 1) + 4 * (gi & 3)) * 2;
        uint32_t va[NO][2];   // this tile's read bases of output tile m, rows vr and vr + 8
#pragma unroll
        for (int m = 0; m < NO; m++)
#pragma unroll
            for (int h = 0; h < 2; h++) va[m][h] = opaque(lds_addr(Vl + tile_off<D, DMA>(vr + 8 * h, 64 * m + vb0, VSTRIDE)));
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int st = 0; st < 2 * NH; st++)
#pragma unroll
            for (int m = 0; m < NO; m++) {
                const f16x8 vb = lds_tr_b16x8_at(va[m][0] + 16 * st * VSTRIDE, va[m][1] + 16 * st * VSTRIDE);
                o[m] = mfma32(pa[st], vb, o[m]);
            }
        // V transpose reads run three MFMAs ahead of their use
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
        for (int j = 0; j < 2 * NH * NO - 3; j++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
        __builtin_amdgcn_s_setprio(0);
    };

    if (c_lo < c_hi) {
        int buf = 0;
        if constexpr (DMA) {
            // tile t + 64 streams into the other buffer while tile t is computed;
            // one barrier per tile: every wave's loads of tile t have landed and
            // every wave is done with the buffer the next loads overwrite
            load_dma(c_lo, lds_k0, lds_v0);
            for (int tile = c_lo; tile < c_hi; tile += PT) {
                __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's loads of tile t
                __syncthreads();
                if (tile + PT < c_hi) load_dma(tile + PT, buf ? lds_k0 : lds_k1, buf ? lds_v0 : lds_v1);
                compute(tile, buf, buf ? lds_k1 : lds_k0, buf ? lds_v1 : lds_v0);
                buf ^= 1;
            }
        } else {
            load_global(c_lo);
            store_lds(0);
            __syncthreads();
            for (int tile = c_lo; tile < c_hi; tile += PT) {
                const bool has_next = tile + PT < c_hi;
                if (has_next) load_global(tile + PT);
                compute(tile, buf, buf ? lds_k1 : lds_k0, buf ? lds_v1 : lds_v0);
                if (has_next) store_lds(buf ^ 1);
                __syncthreads();
                buf ^= 1;
            }
        }
    }

    if (!wave_live) return;
    const float lt = l_run + __shfl_xor(l_run, 32);   // row sum of query row n
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int rr = 8 * (r >> 2) + 4 * hh + (r & 3);   // row of register r
        const float lr = __shfl(lt, rr);
        const int row = Rw + rr;
        if (row < M) {
            const int t = q0 + row / p.gqa, h = hk * p.gqa + row % p.gqa;
            const float inv = lr > 0.f ? 1.f / lr : 0.f;
            float *op = p.out + ((int64_t) t * p.H + h) * D + n;
#pragma unroll
            for (int m = 0; m < NO; m++) op[32 * m] = o[m][r] * inv;
        }
    }
}

template <int D, int NW, int KVT, bool MIXED>
static hipError_t launch_prefill_t(const AttnParams &p, int max_rows, hipStream_t stream) {
    constexpr int ROWS = NW * 32;
    const int n_rb = (max_rows + ROWS - 1) / ROWS;
    const int pairs_per_xcd = (p.S * p.Hkv + 7) / 8;
    const int64_t n_pf = 8 * (int64_t) pairs_per_xcd * n_rb;
    const int64_t n_dec = MIXED ? ((p.sk_workers + NW - 1) / NW + 7) / 8 * 8 : 0;
    const int64_t nwg = n_dec + n_pf;
    if (nwg > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((pa_prefill_kernel<D, NW, KVT, MIXED>), dim3((unsigned) nwg), dim3(NW * 64), 0, stream, p, n_rb,
                       (int) n_dec);
    return hipGetLastError();
}

template <int KVT>
static hipError_t launch_prefill_kv(const AttnParams &p, int head_dim, int max_rows, hipStream_t stream) {
    switch (head_dim) {
        case 64: return launch_prefill_t<64, 4, KVT, false>(p, max_rows, stream);
        case 128: return launch_prefill_t<128, 4, KVT, false>(p, max_rows, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_mixed_f16(const AttnParams &p, int head_dim, int max_rows, hipStream_t stream) {
    switch (head_dim) {
        case 64: return launch_prefill_t<64, 4, 1, true>(p, max_rows, stream);
        case 96: return launch_prefill_t<96, 4, 1, true>(p, max_rows, stream);
        case 128: return launch_prefill_t<128, 4, 1, true>(p, max_rows, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_prefill(const AttnParams &p, int head_dim, int kv_type, int max_rows, hipStream_t stream) {
    if (head_dim == 256) return launch_prefill16(p, head_dim, kv_type, max_rows, stream);
    // f16 pools at head size 64, 96 and 128 take launch_mixed_f16, with or
    // without decode rows
    return kv_type == 8 ? launch_prefill_kv<8>(p, head_dim, max_rows, stream) : hipErrorInvalidValue;
}

}  // namespace iian_pa

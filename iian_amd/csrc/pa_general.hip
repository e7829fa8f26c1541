// pa_general.hip - paged attention for every pool-type and head-size combination
// the MFMA kernels are not built for: F32 pools, mixed K/V types (F32, F16,
// Q8_0 in any pairing), any head size from 1 to 1024 (Phi-3's 96, 80, ...;
// Q8_0 pools in multiples of 32), Dv != D, and block sizes that are not a
// power of two >= 8.  Head sizes that are not multiples of 4 are staged in
// LDS rows padded with zeros to the next multiple of 4 (the reference's
// dot and axpy loops run to any D, paged_attn.cpp:39,50), with element-wise
// global loads and stores, since their rows are not 16-byte aligned.
//
// The arithmetic is fp32 throughout, as in the reference's Kern<float> and
// Kern<fp16> (src/iian/paged_attn.cpp:25-87): K and V are widened to fp32 when
// they are staged (f16 exactly; Q8_0 as q * fp32(d), exactly as
// dequantize_row_q8_0, ggml-quants.c:553-567), scores are fp32 dot products
// with the raw fp32 q, scaled after the dot (paged_attn.cpp:126), softcapped
// as paged_attn.cpp:127, and P and V meet in fp32 FMAs.  F32 pools therefore
// keep their full precision; nothing is narrowed to f16.
//
// Work split.  A workgroup of 4 waves owns 4*RPW query rows of one (sequence,
// kv head): rows r = j*gqa + g (query token j, head g of the GQA group), RPW
// per wave (4, or 1 when no sequence has more than 4 rows per kv head, so
// that decode calls keep all 4 waves busy), and the group shares every
// staged K/V tile.  It attends one of the
// row block's n_split equal ranges of TC-cell tiles (TC = 32, 16 or 8 as the
// head sizes grow, so a tile stays near 16 KB per tensor).  With n_split = 1
// the workgroup writes the normalised output rows; otherwise each range
// writes an unnormalised record (O, m, l) per row and pa_general_merge_kernel
// combines them with a log-sum-exp merge.
//
// Per tile: the rows of its TC cells are looked up once through the block
// table (any block size: cell = table[i / bs] * bs + i % bs,
// include/iian/kv_cache.h:135-137), the table entries read two tiles ahead so
// that no tile waits on them; every thread loads its quads (4 consecutive
// elements) of the next tile into registers while the current tile is
// computed from LDS, then widens them to fp32 into LDS.
//
//   S = Q K^T   lane (c, j) of a wave: cell c of the tile, dims 4j, 4j + 4P,
//               ... (P = 64/TC lanes per cell), for the wave's rows; the P
//               partial sums are added with xor shuffles
//   softmax     online, exp2 domain, per row; masks as paged_attn.cpp:124
//   O += P V    lane owns output dims 4l .. 4l+3 (and 256 + 4l ..) of the
//               wave's rows; P comes from LDS as one broadcast float4 per
//               cell (one float at RPW = 1).  At Dv <= 128 lanes l and l + 32
//               own the same dims over the two halves of the tile's cells
//
// Semantics: paged_attn_impl (src/iian/paged_attn.cpp:90-146), all-masked rows
// -> zeros (:132).
#include "pa_common.h"
#include "pa_launch.h"

namespace iian_pa {

namespace {

constexpr int kGenWaves = 4;
constexpr int kGenMaxRows = kGenWaves * 4;   // rows per workgroup at RPW = 4
constexpr int kGenMaxTile = 32;
constexpr int kGenOutChunks = 4;   // output quads per lane: Dv up to 4 * 64 * 4 = 1024

// Raw bytes of 4 consecutive elements e .. e+3 (e % 4 == 0) of head slice
// `head` of pool row `row`; zeros for row < 0 (a cell beyond the sequence,
// which must stage as 0 so that P = 0 never meets a non-finite V).
// elem: dim is not a multiple of 4, so the quad is loaded element by element
// (the slice is not 16-byte aligned) and its elements at dim and beyond are 0.
template <int TY>
__device__ __forceinline__ u32x4 gen_load(const char *pool, int64_t row, int64_t row_bytes, int head, int dim,
                                          int e, bool elem) {
    u32x4 r = {0u, 0u, 0u, 0u};
    if (row < 0) return r;
    const char *base = pool + row * row_bytes;
    if constexpr (TY == 0) {
        const uint32_t *src = (const uint32_t *) (base + ((int64_t) head * dim + e) * 4);
        if (!elem) {
            r = *(const u32x4 *) src;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) r[j] = e + j < dim ? src[j] : 0u;
        }
    } else if constexpr (TY == 1) {
        const uint16_t *src = (const uint16_t *) (base + ((int64_t) head * dim + e) * 2);
        if (!elem) {
            const u32x2 x = *(const u32x2 *) src;
            r[0] = x[0];
            r[1] = x[1];
        } else {
            uint32_t h[4];
#pragma unroll
            for (int j = 0; j < 4; j++) h[j] = e + j < dim ? src[j] : 0u;
            r[0] = h[0] | (h[1] << 16);
            r[1] = h[2] | (h[3] << 16);
        }
    } else {
        // Q8_0: block e/32 of the head slice is {f16 d, int8 q[32]} (ggml-common.h:251-256);
        // the 4 quants sit 2-byte aligned at 2 + e%32
        const char *blk = base + (int64_t) head * (dim / 32) * 34 + 34 * (e >> 5);
        const uint16_t *qp = (const uint16_t *) (blk + 2 + (e & 31));
        r[0] = (uint32_t) qp[0] | ((uint32_t) qp[1] << 16);
        r[1] = *(const uint16_t *) blk;
    }
    return r;
}

// fp32 values of a quad from gen_load: exact widening (f16), q * fp32(d) (Q8_0).
template <int TY>
__device__ __forceinline__ float4 gen_widen(const u32x4 &r) {
    if constexpr (TY == 0) {
        return make_float4(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[2]),
                           __uint_as_float(r[3]));
    } else if constexpr (TY == 1) {
        const _Float16 a = __builtin_bit_cast(_Float16, (uint16_t) r[0]);
        const _Float16 b = __builtin_bit_cast(_Float16, (uint16_t) (r[0] >> 16));
        const _Float16 c = __builtin_bit_cast(_Float16, (uint16_t) r[1]);
        const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t) (r[1] >> 16));
        return make_float4((float) a, (float) b, (float) c, (float) d);
    } else {
        const float d = (float) __builtin_bit_cast(_Float16, (uint16_t) r[1]);
        return make_float4((float) (int8_t) (r[0]) * d, (float) (int8_t) (r[0] >> 8) * d,
                           (float) (int8_t) (r[0] >> 16) * d, (float) (int8_t) (r[0] >> 24) * d);
    }
}

__device__ __forceinline__ float gen_row_sum(float v, int tc) {
    for (int o = 1; o < tc; o <<= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float gen_row_max(float v, int tc) {
    for (int o = 1; o < tc; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// An output quad at dst holding its row's elements e .. e+3, `left` of them
// (from e) inside the row; elem: element by element (the row is not 16-byte
// aligned), writing only those inside.
__device__ __forceinline__ void gen_store(float *dst, int left, bool elem, const float4 &v) {
    if (!elem) {
        *(float4 *) dst = v;
        return;
    }
    dst[0] = v.x;
    if (left > 1) dst[1] = v.y;
    if (left > 2) dst[2] = v.z;
    if (left > 3) dst[3] = v.w;
}

}  // namespace

// Dynamic LDS: K tile [TC][D4+4] f32 | V tile [TC][Dv4+4] f32 | q [4*RPW][D4] f32 |
// P [4 waves][TC][RPW rows] f32, with D4, Dv4 the head sizes rounded up to a
// multiple of 4 (the padding holds zeros).  The +4 pad spreads the cells of a
// QK^T read over the banks.
// RPW rows per wave.  At RPW = 1 (decode calls) the register allocator is
// asked for three waves per SIMD (at most 168 VGPRs): three 4-wave workgroups
// per CU.  Four (128 VGPRs, 2 spilled) measured 1.5% faster at cfg2's shape
// with F32 pools; left at three.
template <int KT, int VT, int RPW>
__global__ __launch_bounds__(kGenWaves * 64, RPW == 1 ? 3 : 1) void pa_general_kernel(GenParams p) {
    constexpr int kGenRowsPerWave = RPW;
    constexpr int kGenRows = kGenWaves * RPW;
    extern __shared__ __attribute__((aligned(16))) float gen_lds[];
    __shared__ int64_t rows_lds[2][kGenMaxTile];

    const int TC = p.tile_cells, D = p.D, Dv = p.Dv;
    const int D4 = (D + 3) & ~3, Dv4 = (Dv + 3) & ~3;
    const bool kelem = (D & 3) != 0, velem = (Dv & 3) != 0;   // rows not 16-byte aligned: element-wise
    const int kst = D4 + 4, vst = Dv4 + 4;
    float *Kl = gen_lds;
    float *Vl = Kl + TC * kst;
    float *Ql = Vl + TC * vst;
    float *Pl = Ql + kGenRows * D4;

    // workgroup -> (pair, row block, split); the splits of one row block are
    // neighbours, and so are the row blocks of one (sequence, kv head)
    const int64_t wid = blockIdx.x;
    const int z = (int) (wid % p.n_split);
    const int64_t rest = wid / p.n_split;
    const int rb = (int) (rest % p.n_rb);
    const int pair = (int) (rest / p.n_rb);
    const int s = pair / p.Hkv, hk = pair % p.Hkv;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int L = max(p.seq_lens[s], 0);
    const int q0 = min(max(p.qsl[s], 0), p.T);
    const int nq = min(max(p.qsl[s + 1], q0), p.T) - q0;
    const int M = nq * p.gqa;
    // a sequence with more query tokens than the caller's max_query_len has
    // rows no workgroup of this launch covers: flag it (bit 2)
    if (rb == 0 && z == 0 && hk == 0 && tid == 0 && nq > p.max_q && p.err) atomicOr(p.err, 4);
    const int R0 = rb * kGenRows;
    if (R0 >= M) return;

    // positions of the workgroup's rows and of this wave's rows
    int wg_min = INT32_MAX, wg_max = INT32_MIN;
    {
        const int j0 = R0 / p.gqa, j1 = (min(M, R0 + kGenRows) - 1) / p.gqa;
        for (int j = j0 + lane; j <= j1; j += 64) {
            const int ps = p.pos[q0 + j];
            wg_min = min(wg_min, ps);
            wg_max = max(wg_max, ps);
        }
        for (int o = 32; o >= 1; o >>= 1) {
            wg_min = min(wg_min, __shfl_xor(wg_min, o));
            wg_max = max(wg_max, __shfl_xor(wg_max, o));
        }
    }
    int prow[kGenRowsPerWave];
    bool rlive[kGenRowsPerWave];
    int w_min = INT32_MAX, w_max = INT32_MIN;
#pragma unroll
    for (int i = 0; i < kGenRowsPerWave; i++) {
        const int r = R0 + wave * kGenRowsPerWave + i;
        rlive[i] = r < M;
        prow[i] = rlive[i] ? p.pos[q0 + r / p.gqa] : 0;
        if (rlive[i]) {
            w_min = min(w_min, prow[i]);
            w_max = max(w_max, prow[i]);
        }
    }
    const bool wave_live = rlive[0];

    // the cells any row of the workgroup can see, and this split's tiles of them
    int c_hi = L;
    if (p.causal) c_hi = min(c_hi, max(wg_max + 1, 0));
    const int c_lo = p.n_swa > 0 ? min(max(0, wg_min - p.n_swa + 1), c_hi) : 0;
    const int nt = (c_hi - c_lo + TC - 1) / TC;
    const int per = (nt + p.n_split - 1) / p.n_split;
    const int t0 = min(nt, z * per), t1 = min(nt, t0 + per);

    // q rows of the workgroup into LDS (raw fp32; the scale follows the dot)
    const int dq = D4 >> 2;
    for (int i = tid; i < kGenRows * dq; i += kGenWaves * 64) {
        const int r = i / dq, c4 = i - r * dq;
        const int rr = R0 + r;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (rr < M) {
            const int t = q0 + rr / p.gqa, h = hk * p.gqa + rr % p.gqa;
            const float *qp = p.q + ((int64_t) t * p.H + h) * D + 4 * c4;
            if (!kelem) {
                v = *(const float4 *) qp;
            } else {
                const int e = 4 * c4;
                v = make_float4(qp[0], e + 1 < D ? qp[1] : 0.f, e + 2 < D ? qp[2] : 0.f, e + 3 < D ? qp[3] : 0.f);
            }
        }
        *(float4 *) (Ql + r * D4 + 4 * c4) = v;
    }

    // pool rows of the TC cells of tile t (by threads 0 .. TC-1), in two
    // steps: tile_bt issues the block-table read two tiles ahead (the entry
    // stays in a register), tile_row turns it into the cell's pool row in LDS
    // one tile later, so no tile waits on a table read
    struct BtEntry {
        int c, b;
        int32_t id;
    };
    auto tile_bt = [&](int t) {
        BtEntry e = {-1, 0, 0};
        if (tid < TC && t < t1) {
            const int c = c_lo + t * TC + tid;
            if (c < c_hi) {
                int b = c / p.block_size;
                if (b >= p.max_blocks) {
                    if (p.err) atomicOr(p.err, 2);
                    b = p.max_blocks - 1;
                }
                e = {c, b, p.bt[(int64_t) s * p.max_blocks + b]};
            }
        }
        return e;
    };
    auto tile_row = [&](const BtEntry &e, int buf) {
        if (tid < TC) {
            int64_t row = -1;
            if (e.c >= 0) {
                int32_t id = e.id;
                if ((uint32_t) id >= (uint32_t) p.num_blocks) {
                    if (p.err) atomicOr(p.err, 2);
                    id = 0;
                }
                row = (int64_t) id * p.block_size + (e.c - e.b * p.block_size);
                if (e.c - e.b * p.block_size >= p.block_size) row = (int64_t) id * p.block_size;   // clamped b
            }
            rows_lds[buf][tid] = row;
        }
    };

    // per-thread quads of one tile: K quads i = tid + 256k of TC*D4/4, V likewise
    const int kq = TC * dq, vq = TC * (Dv4 >> 2);
    u32x4 kraw[4], vraw[4];
    auto load_tile = [&](int buf) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = tid + k * kGenWaves * 64;
            if (i < kq) {
                const int c = i / dq, e = 4 * (i - c * dq);
                kraw[k] = gen_load<KT>(p.k_pool, rows_lds[buf][c], p.k_row, hk, D, e, kelem);
            }
            if (i < vq) {
                const int c = i / (Dv4 >> 2), e = 4 * (i - c * (Dv4 >> 2));
                vraw[k] = gen_load<VT>(p.v_pool, rows_lds[buf][c], p.v_row, hk, Dv, e, velem);
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = tid + k * kGenWaves * 64;
            if (i < kq) {
                const int c = i / dq, e = 4 * (i - c * dq);
                *(float4 *) (Kl + c * kst + e) = gen_widen<KT>(kraw[k]);
            }
            if (i < vq) {
                const int c = i / (Dv4 >> 2), e = 4 * (i - c * (Dv4 >> 2));
                *(float4 *) (Vl + c * vst + e) = gen_widen<VT>(vraw[k]);
            }
        }
    };

    const int P = 64 / TC;                 // lanes per cell in QK^T
    const int cl = lane % TC, jl = lane / TC;
    const int ndv = Dv4 >> 2;              // output quads per row
    // Dv <= 128: a row's output quads fill half a wave, so the two lane halves
    // take the two halves of the tile's cells in PV and add their sums at the end
    const bool pv_halves = ndv <= 32;
    const int pv_lane = pv_halves ? (lane & 31) : lane;
    const int pv_c0 = pv_halves ? (lane >> 5) * (TC >> 1) : 0, pv_c1 = pv_halves ? pv_c0 + (TC >> 1) : TC;
    float m_run[kGenRowsPerWave], l_run[kGenRowsPerWave];
    float4 o[kGenRowsPerWave][kGenOutChunks];
#pragma unroll
    for (int i = 0; i < kGenRowsPerWave; i++) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.f;
#pragma unroll
        for (int k = 0; k < kGenOutChunks; k++) o[i][k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float *Pw = Pl + wave * TC * RPW;

    auto compute = [&](int t) {
        const int base = c_lo + t * TC;
        if (!wave_live) return;
        if (p.causal && base > w_max) return;                          // after every row of the wave
        if (p.n_swa > 0 && base + TC - 1 <= w_min - p.n_swa) return;   // out of every row's window
        // scores of cell cl for the wave's rows
        float acc[kGenRowsPerWave] = {};
        const float *kr = Kl + cl * kst;
        const float *qr = Ql + wave * kGenRowsPerWave * D4;
        for (int d = 4 * jl; d < D4; d += 4 * P) {
            const float4 k4 = *(const float4 *) (kr + d);
#pragma unroll
            for (int i = 0; i < kGenRowsPerWave; i++) {
                const float4 q4 = *(const float4 *) (qr + i * D4 + d);
                acc[i] = fmaf(q4.x, k4.x, acc[i]);
                acc[i] = fmaf(q4.y, k4.y, acc[i]);
                acc[i] = fmaf(q4.z, k4.z, acc[i]);
                acc[i] = fmaf(q4.w, k4.w, acc[i]);
            }
        }
        const int c = base + cl;
        float pv[kGenRowsPerWave], alpha[kGenRowsPerWave];
#pragma unroll
        for (int i = 0; i < kGenRowsPerWave; i++) {
            for (int off = TC; off < 64; off <<= 1) acc[i] += __shfl_xor(acc[i], off);
            float sc = acc[i] * p.scale;
            if (p.softcap > 0.f) sc = p.softcap * tanhf(sc / p.softcap);
            const bool vis = rlive[i] && c < c_hi && (!p.causal || c <= prow[i]) &&
                             (p.n_swa <= 0 || prow[i] - c < p.n_swa);
            const float x = vis ? sc * kLog2e : -INFINITY;
            const float mt = gen_row_max(x, TC);
            const float mnew = fmaxf(m_run[i], mt);
            if (mnew == -INFINITY) {
                alpha[i] = 1.f;
                pv[i] = 0.f;
            } else {
                alpha[i] = __builtin_amdgcn_exp2f(m_run[i] - mnew);
                pv[i] = __builtin_amdgcn_exp2f(x - mnew);
            }
            m_run[i] = mnew;
            l_run[i] = l_run[i] * alpha[i] + gen_row_sum(pv[i], TC);
        }
        if (jl == 0) {
            if constexpr (RPW == 4) {
                *(float4 *) (Pw + 4 * cl) = make_float4(pv[0], pv[1], pv[2], pv[3]);
            } else {
#pragma unroll
                for (int i = 0; i < RPW; i++) Pw[RPW * cl + i] = pv[i];
            }
        }
        lds_barrier<1>();   // this wave's P stores before its reads (no s_barrier)
#pragma unroll
        for (int i = 0; i < kGenRowsPerWave; i++)
#pragma unroll
            for (int k = 0; k < kGenOutChunks; k++) {
                o[i][k].x *= alpha[i];
                o[i][k].y *= alpha[i];
                o[i][k].z *= alpha[i];
                o[i][k].w *= alpha[i];
            }
#pragma unroll
        for (int k = 0; k < kGenOutChunks; k++) {
            const int d4 = pv_lane + 64 * k;
            if (d4 >= ndv) break;
            const float *vc = Vl + 4 * d4;
            for (int cc = pv_c0; cc < pv_c1; cc++) {
                const float4 v4 = *(const float4 *) (vc + cc * vst);
                float pr[RPW];
                if constexpr (RPW == 4) {
                    const float4 pp = *(const float4 *) (Pw + 4 * cc);
                    pr[0] = pp.x;
                    pr[1] = pp.y;
                    pr[2] = pp.z;
                    pr[3] = pp.w;
                } else {
#pragma unroll
                    for (int i = 0; i < RPW; i++) pr[i] = Pw[RPW * cc + i];
                }
#pragma unroll
                for (int i = 0; i < kGenRowsPerWave; i++) {
                    o[i][k].x = fmaf(pr[i], v4.x, o[i][k].x);
                    o[i][k].y = fmaf(pr[i], v4.y, o[i][k].y);
                    o[i][k].z = fmaf(pr[i], v4.z, o[i][k].z);
                    o[i][k].w = fmaf(pr[i], v4.w, o[i][k].w);
                }
            }
        }
        lds_barrier<1>();   // P reads done before the next tile's P stores
    };

    if (t0 < t1) {
        tile_row(tile_bt(t0), 0);
        BtEntry next = tile_bt(t0 + 1);
        __syncthreads();
        load_tile(0);
        for (int t = t0; t < t1; t++) {
            const int buf = (t - t0) & 1;
            __syncthreads();   // every wave is done with the K/V tile in LDS
            store_tile();
            if (t + 1 < t1) tile_row(next, buf ^ 1);
            next = tile_bt(t + 2);
            __syncthreads();
            if (t + 1 < t1) load_tile(buf ^ 1);
            compute(t);
        }
    }

    if (!wave_live) return;
    if (pv_halves) {   // lanes l and l + 32 hold the two cell halves' sums of the same quad
#pragma unroll
        for (int i = 0; i < kGenRowsPerWave; i++) {
            o[i][0].x += __shfl_xor(o[i][0].x, 32);
            o[i][0].y += __shfl_xor(o[i][0].y, 32);
            o[i][0].z += __shfl_xor(o[i][0].z, 32);
            o[i][0].w += __shfl_xor(o[i][0].w, 32);
        }
    }
#pragma unroll
    for (int i = 0; i < kGenRowsPerWave; i++) {
        if (!rlive[i]) continue;
        const int r = R0 + wave * kGenRowsPerWave + i;
        const int t = q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
        const int64_t orow = (int64_t) t * p.H + h;
        if (p.n_split == 1) {
            const float inv = l_run[i] > 0.f ? 1.f / l_run[i] : 0.f;
#pragma unroll
            for (int k = 0; k < kGenOutChunks; k++) {
                const int d4 = lane + 64 * k;
                if (d4 < ndv)
                    gen_store(p.out + orow * Dv + 4 * d4, Dv - 4 * d4, velem,
                              make_float4(o[i][k].x * inv, o[i][k].y * inv, o[i][k].z * inv, o[i][k].w * inv));
            }
        } else {
            // records are Dv4 floats a row, so every quad stays aligned
            const int64_t rec = orow * p.n_split + z;
#pragma unroll
            for (int k = 0; k < kGenOutChunks; k++) {
                const int d4 = lane + 64 * k;
                if (d4 < ndv) *(float4 *) (p.part_o + rec * Dv4 + 4 * d4) = o[i][k];
            }
            if (lane == 0) *(float2 *) (p.part_ml + 2 * rec) = make_float2(m_run[i], l_run[i]);
        }
    }
}

// Log-sum-exp merge of the n_split records of every output row (one wave per
// row): out = sum_j 2^(m_j - m) O_j / sum_j 2^(m_j - m) l_j, m = max_j m_j.  A
// record with m_j = -inf (a range with no visible cell, or no tile at all) is
// skipped, so its O is never read.
__global__ __launch_bounds__(256) void pa_general_merge_kernel(GenParams p) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t) blockIdx.x * 4 + wave;
    if (row >= (int64_t) p.T * p.H) return;
    const int ns = p.n_split;
    // rows of a sequence past the launch's row blocks have no records
    const int t = (int) (row / p.H), h = (int) (row % p.H);
    int s = 0;
    {
        int lo = 0, hi = p.S - 1;   // last s with qsl[s] <= t
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (p.qsl[mid] <= t) lo = mid; else hi = mid - 1;
        }
        s = lo;
    }
    const int j = t - p.qsl[s];
    if (j < 0 || (j * p.gqa + h % p.gqa) >= p.n_rb * p.rows_per_block) return;
    const float2 ml = lane < ns ? *(const float2 *) (p.part_ml + 2 * (row * ns + lane)) : make_float2(-INFINITY, 0.f);
    const float mx = wave_max(gen_row_max(ml.x, 16));
    const int Dv4 = (p.Dv + 3) & ~3;
    const bool velem = (p.Dv & 3) != 0;
    const int ndv = Dv4 >> 2;
    float4 acc[kGenOutChunks];
#pragma unroll
    for (int k = 0; k < kGenOutChunks; k++) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    float lsum = 0.f;
    if (mx != -INFINITY) {
        const float w = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
        lsum = w * ml.y;
        for (int o = 1; o < 64; o <<= 1) lsum += __shfl_xor(lsum, o);
        for (int r = 0; r < ns; r++) {
            const float wr = __shfl(w, r);
            if (wr == 0.f) continue;   // wave-uniform
            const float *op = p.part_o + (row * ns + r) * Dv4;
#pragma unroll
            for (int k = 0; k < kGenOutChunks; k++) {
                const int d4 = lane + 64 * k;
                if (d4 < ndv) {
                    const float4 v = *(const float4 *) (op + 4 * d4);
                    acc[k].x = fmaf(wr, v.x, acc[k].x);
                    acc[k].y = fmaf(wr, v.y, acc[k].y);
                    acc[k].z = fmaf(wr, v.z, acc[k].z);
                    acc[k].w = fmaf(wr, v.w, acc[k].w);
                }
            }
        }
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
    for (int k = 0; k < kGenOutChunks; k++) {
        const int d4 = lane + 64 * k;
        if (d4 < ndv)
            gen_store(p.out + row * p.Dv + 4 * d4, p.Dv - 4 * d4, velem,
                      make_float4(acc[k].x * inv, acc[k].y * inv, acc[k].z * inv, acc[k].w * inv));
    }
}

size_t general_lds_bytes(int tile_cells, int D, int Dv, int rows_per_block) {
    const size_t D4 = (size_t) (D + 3) & ~(size_t) 3, Dv4 = (size_t) (Dv + 3) & ~(size_t) 3;
    return ((size_t) tile_cells * (D4 + 4) + (size_t) tile_cells * (Dv4 + 4) + (size_t) rows_per_block * D4 +
            (size_t) tile_cells * rows_per_block) *
           sizeof(float);
}

// Cells per tile: a tile's quads of each tensor stay within 4 per thread
// (TC * D4 / 4 <= 1024), and its LDS below 100 KB at head size 1024.
int general_tile_cells(int D, int Dv) {
    const int m = D > Dv ? D : Dv;
    return m <= 128 ? 32 : (m <= 256 ? 16 : (m <= 512 ? 8 : 4));
}

// Rows per workgroup: 4 (one per wave) when no sequence of the call has more
// than 4 rows per kv head, else 16.
int general_rows_per_block(int max_rows) { return max_rows <= kGenWaves ? kGenWaves : kGenMaxRows; }

template <int KT, int VT, int RPW>
static hipError_t launch_general_r(const GenParams &p, hipStream_t stream) {
    const size_t lds = general_lds_bytes(p.tile_cells, p.D, p.Dv, kGenWaves * RPW);
    const int64_t nwg = (int64_t) p.S * p.Hkv * p.n_rb * p.n_split;
    if (nwg <= 0 || nwg > INT32_MAX) return hipErrorInvalidValue;
    if (lds > 64 * 1024) {   // head sizes above 256: more than 64 KB of dynamic LDS needs the opt-in
        const hipError_t e = hipFuncSetAttribute((const void *) pa_general_kernel<KT, VT, RPW>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((pa_general_kernel<KT, VT, RPW>), dim3((unsigned) nwg), dim3(kGenWaves * 64), lds, stream, p);
    return hipGetLastError();
}

template <int KT, int VT>
static hipError_t launch_general_t(const GenParams &p, hipStream_t stream) {
    hipError_t e = p.rows_per_block == kGenWaves ? launch_general_r<KT, VT, 1>(p, stream)
                                                 : launch_general_r<KT, VT, 4>(p, stream);
    if (e != hipSuccess || p.n_split == 1) return e;
    const int64_t rows = (int64_t) p.T * p.H;
    hipLaunchKernelGGL(pa_general_merge_kernel, dim3((unsigned) ((rows + 3) / 4)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <int KT>
static hipError_t launch_general_k(const GenParams &p, int type_v, hipStream_t stream) {
    switch (type_v) {
        case 0: return launch_general_t<KT, 0>(p, stream);
        case 1: return launch_general_t<KT, 1>(p, stream);
        case 8: return launch_general_t<KT, 8>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_general(const GenParams &p, int type_k, int type_v, hipStream_t stream) {
    switch (type_k) {
        case 0: return launch_general_k<0>(p, type_v, stream);
        case 1: return launch_general_k<1>(p, type_v, stream);
        case 8: return launch_general_k<8>(p, type_v, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iian_pa

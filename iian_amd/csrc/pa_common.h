// pa_common.h - shared device-side types and helpers of the gfx950 paged-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iian_pa {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTile = 32;   // cells per KV tile (two 16-row MFMA halves)
// Lazy online-softmax rescale: a row's reference max moves only when a tile
// max exceeds it by more than this (log2 units), so P stays <= 2^8 in f16.
constexpr float kRescaleSlack = 8.0f;
// Sequences with n_q*gqa up to this many rows per kv head run through the decode kernels.
constexpr int kDecodeRowsMax = 32;

// Everything the attention kernels read, by value (kernel argument segment).
struct AttnParams {
    const float *q;             // [T][H][D]
    const char *k_pool;         // cell rows of Hkv*D elements
    const char *v_pool;
    const int32_t *bt;          // [S][max_blocks]
    const int32_t *seq_lens;    // [S]
    const int32_t *qsl;         // [S+1]
    const int32_t *pos;         // [T]
    float *out;                 // [T][H][Dv]
    float *part_o;              // stream-K partial records: numerators, rec_stride floats per record
    float *part_ml;             // (reference max in log2 units, sum) per record row
    int2 *seg_info;             // per segment: (first record, pieces), written by the segment's first piece
    uint64_t *seg_ctr;          // per (sequence, kv head): (call epoch << 16) | pieces counted in (mixed launch)
    int32_t *err;               // nullable error word
    const float *k_new;         // iian_pa_write_attention: the step's new K rows, f32 [T][Hkv*D] (else null)
    const float *v_new;         // and V rows, f32 [T][Hkv*Dv]
    int64_t k_row;              // bytes per K pool row (< 2^32)
    int64_t v_row;              // equal to k_row: K and V share type and head size
    int64_t rec_stride;         // floats per record of part_o
    uint64_t epoch;             // this call's tag for seg_ctr (48 bits)
    int32_t max_blocks;
    int32_t num_blocks;
    int32_t T, S, H, Hkv, gqa;
    int32_t bs_log2;
    float qscale;               // folded into q before the f16 conversion
    float softcap;              // 0 = off
    float softcap_inv;
    int32_t causal;
    int32_t n_swa;
    int32_t decode_rows;        // sequences with n_q*gqa <= decode_rows use the decode kernel
    int32_t max_q;              // the caller's max_query_len (a sequence with more tokens sets err bit 2)
    int32_t sk_workers;         // stream-K workers: waves (one kv head each) or groups of Hkv workgroups
    int32_t rec_heads;          // kv heads per partial record: 1, or Hkv for grouped workers
    int32_t seg_waves;          // > 0: f16 decode by pa_decode_seg_kernel, seg_waves waves per segment
    int32_t cus_per_xcd;        // CUs per XCD: workgroups b and b + 8*cus_per_xcd of a launch share a CU
    int32_t head_group;         // kv heads per f16 decode segment: 1, or 2 (head size 96, rows per head <= 8)
    int32_t rec_rows;           // rows of a partial record per kv-head slot: decode_rows * head_group
};

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

// Physical block id of logical block b of sequence s, clamped into the table
// row and the pool (a seq_len beyond the table's capacity or a stale block id
// is flagged, never dereferenced).
__device__ __forceinline__ int32_t phys_block(const AttnParams &p, int s, int b) {
    if (b >= p.max_blocks) {
        if (p.err) atomicOr(p.err, 2);
        b = p.max_blocks - 1;
    }
    int32_t id = p.bt[(int64_t) s * p.max_blocks + b];
    if ((uint32_t) id >= (uint32_t) p.num_blocks) {
        if (p.err) atomicOr(p.err, 2);
        id = 0;
    }
    return id;
}

// ---- Stream-K partition of the decode work ----
//
// A decode sequence (1 <= n_q and n_q*gqa <= decode_rows query rows) attends
// the window [c_lo, c_hi) of cells that any of its query positions can see
// (causal and sliding-window bounds; c_lo a multiple of kTile).  Its window is
// nt = max(1, ceil((c_hi - c_lo)/kTile)) tiles: an empty window keeps one tile,
// whose piece writes the zero rows of paged_attn.cpp:132.  Laid end to end in
// sequence order, the windows form one line of tiles; a segment is a
// (sequence, kv head) stretch of it when each worker is one wave of one kv head
// (UNIT = Hkv segments per sequence), or a whole sequence when a worker is a
// group of Hkv workgroups, one per kv head (UNIT = 1).  Worker w takes line
// tiles [w*per, (w+1)*per) with per = ceil(total / workers), whatever
// sequences they fall in, so every worker carries the same work however ragged
// the contexts are.  The stretch of one worker inside one segment is a piece;
// a segment with one piece writes its output directly, the others write
// partial records merged by pa_merge_kernel (or, in the mixed prefill launch,
// by the segment's last piece to finish: arrive_last).  Piece (worker w, segment seg) has
// record w + seg: along the line either w or seg grows by one from piece to
// piece, so records are unique and a segment's pieces hold consecutive ones.
constexpr int kMinPieceTiles = 2;

struct SeqWindow {
    int L, q0, nq;
    int pmin, pmax;
    int c_lo, c_hi;   // [c_lo, c_hi): c_lo a multiple of kTile
    int nt;           // tiles of the window; 0 when s is not a decode sequence
};

// Window of sequence s (s >= S, or not a decode sequence: nt = 0).  Called
// per lane (one sequence each) to count tiles, and with a wave-uniform s
// (scalar loads) for the sequence of a piece.
__device__ __forceinline__ SeqWindow seq_window(const AttnParams &p, int s) {
    SeqWindow w = {0, 0, 0, 0, 0, 0, 0, 0};
    if (s >= p.S) return w;
    w.L = max(p.seq_lens[s], 0);
    w.q0 = min(max(p.qsl[s], 0), p.T);
    w.nq = min(max(p.qsl[s + 1], w.q0), p.T) - w.q0;
    if (w.nq <= 0 || w.nq * p.gqa > p.decode_rows) return w;
    int mn = INT32_MAX, mx = INT32_MIN;
    for (int i = 0; i < w.nq; i++) {
        const int ps = p.pos[w.q0 + i];
        mn = min(mn, ps);
        mx = max(mx, ps);
    }
    w.pmin = mn;
    w.pmax = mx;
    int hi = w.L;
    if (p.causal) hi = min(hi, max(w.pmax + 1, 0));
    int lo = 0;
    if (p.n_swa > 0) lo = max(0, w.pmin - p.n_swa + 1);
    lo &= ~(kTile - 1);
    if (hi < lo) hi = lo;
    w.c_lo = lo;
    w.c_hi = hi;
    w.nt = max(1, (hi - lo + kTile - 1) / kTile);
    return w;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    return v;
}

// One piece of a worker's range: sequence s (window w), kv head hk, window
// tiles [t0, t1), partial record rec, the segment's first record rec0 and its
// piece count (1 = the piece is the whole segment and writes the output itself).
struct Piece {
    int s, hk, t0, t1, rec, rec0, pieces, seg;
};

// Calls body(w, piece) for each piece of worker `worker` (wave-uniform).
// GROUPED: one segment per sequence and the worker's kv head is hk_fixed;
// otherwise segments are (sequence, kv head).
template <bool GROUPED, typename Body>
__device__ __forceinline__ void for_each_piece(const AttnParams &p, int worker, int hk_fixed, Body &&body) {
    const int lane = threadIdx.x & 63;
    const int unit = GROUPED ? 1 : p.Hkv / p.head_group;   // segments per sequence
    // lanes hold the tile counts of sequences base + lane and their inclusive
    // prefix along the line; a piece's window is re-read with scalar loads
    // (keeping every field in lanes costs registers the tile loop needs)
    SeqWindow w0 = seq_window(p, lane);
    int nt = w0.nt;
    int total = wave_sum_i(nt);
    bool over = w0.nq > p.max_q;
    for (int b = 64; b < p.S; b += 64) {
        const SeqWindow wb = seq_window(p, b + lane);
        total += wave_sum_i(wb.nt);
        over |= wb.nq > p.max_q;
    }
    // a sequence with more query tokens than the caller's max_query_len may
    // have rows this launch does not cover: worker 0 flags it (bit 2)
    if (worker == 0 && __builtin_amdgcn_ballot_w64(over) && lane == 0 && p.err) atomicOr(p.err, 4);
    total = __builtin_amdgcn_readfirstlane(total) * unit;
    const int per = max(kMinPieceTiles, (total + p.sk_workers - 1) / p.sk_workers);
    int start = worker * per;
    const int end = min(total, start + per);
    if (start >= end) return;
    int base = 0;
    int incl = wave_incl_scan(nt * unit);
    for (;;) {
        uint64_t hit = __builtin_amdgcn_ballot_w64(incl > start);
        while (!hit) {   // the next sequence with tiles lies beyond these 64
            const int carry = __shfl(incl, 63);
            base += 64;
            nt = seq_window(p, base + lane).nt;
            incl = carry + wave_incl_scan(nt * unit);
            hit = __builtin_amdgcn_ballot_w64(incl > start);
        }
        const int ls = __builtin_ctzll(hit);
        const int s = base + ls;
        const SeqWindow w = seq_window(p, s);
        const int excl = __builtin_amdgcn_readfirstlane(__shfl(incl, ls)) - w.nt * unit;
        const int off = start - excl;
        Piece pc;
        pc.s = s;
        pc.hk = GROUPED ? hk_fixed : off / w.nt;
        pc.t0 = GROUPED ? off : off % w.nt;
        pc.t1 = min(w.nt, pc.t0 + (end - start));
        const int seg_start = excl + (GROUPED ? 0 : pc.hk * w.nt);
        pc.seg = GROUPED ? s : s * unit + pc.hk;
        pc.rec = worker + pc.seg;
        pc.rec0 = seg_start / per + pc.seg;   // record of the segment's first piece
        pc.pieces = (seg_start + w.nt - 1) / per - seg_start / per + 1;
        body(w, pc);
        start = seg_start + pc.t1;
        if (start >= end) break;
    }
}

// Partial record row r of kv head slot hr (0, or the kv head for grouped workers).
__device__ __forceinline__ float *rec_o(const AttnParams &p, int rec, int hr, int r, int dv) {
    return p.part_o + (int64_t) rec * p.rec_stride + ((int64_t) hr * p.rec_rows + r) * dv;
}
__device__ __forceinline__ float *rec_ml(const AttnParams &p, int rec, int hr, int r) {
    return p.part_ml + (((int64_t) rec * p.rec_heads + hr) * p.rec_rows + r) * 2;
}

// ---- Merge of a split segment inside the launch (mixed prefill launch) ----
//
// The L2s of MI355X's XCDs are not coherent with each other within a launch,
// so the partial records are handed over in agent-scope operations: stores
// and loads with the sc1 bit (written through to, and read from, the
// device-coherent level).  A piece writes its record rows that way, waits for
// them (s_waitcnt vmcnt(0)), then counts itself in on the segment's counter
// (arrive_last); the piece that completes the count reads every record of the
// segment with agent-scope loads and writes the output.  No release fence is
// needed (on gfx950 an agent-scope release writes back the whole L2):
// everything handed over travels in agent-scope operations, and the wait
// orders them before the count.  The chain of memory round trips this puts
// after a worker's last piece costs more than a merge launch when the decode
// kernel runs alone, so only the mixed launch merges this way: there the
// decode workers finish long before the prefill workgroups.
__device__ __forceinline__ void store_pair_agent(float *ptr, float a, float b) {   // ptr 8-byte aligned
    const uint64_t v = (uint64_t) __float_as_uint(a) | ((uint64_t) __float_as_uint(b) << 32);
    __hip_atomic_store((uint64_t *) ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_pair_agent(const float *ptr) {
    const uint64_t v = __hip_atomic_load((uint64_t *) ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t) v), __uint_as_float((uint32_t) (v >> 32)));
}

// Counts the calling wave in on counter ctr after its record stores have
// completed; true (wave-uniform) for the wave that brings the count to
// `expected`.  A counter holding another epoch (another call, or workspace
// bytes never written by this library) counts as zero, so the workspace needs
// no initialisation.  The completing wave resets the counter to (epoch, 0),
// which keeps replays of a captured launch, which reuse one epoch, correct.
// The compare-and-swap loop ends: each failed attempt means another wave's
// attempt succeeded, and at most `expected` waves use the counter per call.
__device__ __forceinline__ bool arrive_last(uint64_t *ctr, uint64_t epoch, int expected) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's record stores are complete
    uint32_t cnt = 0;
    if ((threadIdx.x & 63) == 0) {
        uint64_t old = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (;;) {
            const uint64_t nw = (old >> 16) == epoch ? old + 1 : (epoch << 16) | 1u;
            if (__hip_atomic_compare_exchange_strong(ctr, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)) {
                cnt = (uint32_t) (nw & 0xffffu);
                break;
            }
        }
        if (cnt == (uint32_t) expected) __hip_atomic_store(ctr, epoch << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    cnt = __builtin_amdgcn_readfirstlane(__shfl(cnt, 0));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // record loads only after the count
    return cnt == (uint32_t) expected;
}

// Log-sum-exp merge of rows [row0, row0 + 16) of kv-head slot hr over the
// segment's records rec0 .. rec0+np-1, written to the output rows of kv head
// hk: out = sum_j 2^(m_j - m) O_j / sum_j 2^(m_j - m) l_j, m = max_j m_j
// (rows every record left at m = -inf are all-masked and come out as zeros).
// Lane (g, n) merges rows row0 + 4g + i, dims (D/16)n .. (D/16)n + D/16 - 1;
// the loads of two records are issued together.
template <int D>
__device__ __forceinline__ void merge_tile16(const AttnParams &p, int rec0, int np, int hr, int row0, int M,
                                             int q0, int hk) {
    constexpr int DPL = D / 16;
    constexpr int B = 2;
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    float mx[4], ls[4], acc[4][DPL];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        mx[i] = -INFINITY;
        ls[i] = 0.f;
#pragma unroll
        for (int d = 0; d < DPL; d++) acc[i][d] = 0.f;
    }
    for (int j0 = 0; j0 < np; j0 += B) {
        float2 ml[B][4], ov[B][4][DPL / 2];
#pragma unroll
        for (int u = 0; u < B; u++) {
            const int j = rec0 + min(j0 + u, np - 1);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = min(row0 + 4 * g + i, M - 1);   // rows >= M are never written
                ml[u][i] = load_pair_agent(rec_ml(p, j, hr, r));
                const float *op = rec_o(p, j, hr, r, D) + DPL * n;
#pragma unroll
                for (int c = 0; c < DPL / 2; c++) ov[u][i][c] = load_pair_agent(op + 2 * c);
            }
        }
#pragma unroll
        for (int u = 0; u < B; u++) {
            if (j0 + u >= np) break;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float mn = fmaxf(mx[i], ml[u][i].x);
                if (mn == -INFINITY) continue;
                const float a = __builtin_amdgcn_exp2f(mx[i] - mn), b = __builtin_amdgcn_exp2f(ml[u][i].x - mn);
                mx[i] = mn;
                ls[i] = ls[i] * a + ml[u][i].y * b;
#pragma unroll
                for (int c = 0; c < DPL / 2; c++) {
                    acc[i][2 * c] = acc[i][2 * c] * a + ov[u][i][c].x * b;
                    acc[i][2 * c + 1] = acc[i][2 * c + 1] * a + ov[u][i][c].y * b;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = row0 + 4 * g + i;
        if (r >= M) continue;
        const int t = q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
        const float inv = ls[i] > 0.f ? 1.f / ls[i] : 0.f;
        float *op = p.out + ((int64_t) t * p.H + h) * D + DPL * n;
        if constexpr (DPL % 4 == 0) {
#pragma unroll
            for (int d = 0; d < DPL; d += 4)
                *(float4 *) (op + d) = make_float4(acc[i][d] * inv, acc[i][d + 1] * inv, acc[i][d + 2] * inv,
                                                   acc[i][d + 3] * inv);
        } else {   // D = 96: 6 dims per lane, 8-byte aligned
#pragma unroll
            for (int d = 0; d < DPL; d += 2) *(float2 *) (op + d) = make_float2(acc[i][d] * inv, acc[i][d + 1] * inv);
        }
    }
}

// Block-table entries of 64 consecutive logical blocks of one sequence, one
// per lane, read once per split and handed out with lane shuffles.
struct TableWindow {
    int first;     // logical block held by lane 0
    int32_t id;    // this lane's physical block id
};

__device__ __forceinline__ void table_load(const AttnParams &p, int s, int first, int L, TableWindow &tw) {
    const int lane = threadIdx.x & 63;
    const int nblk = (L + (1 << p.bs_log2) - 1) >> p.bs_log2;
    tw.first = first;
    tw.id = (first + lane < nblk) ? phys_block(p, s, first + lane) : 0;
}

// Pool row of cell c (c <= L-1) whose 8-cell group starts at grp (grp <= c, same block).
__device__ __forceinline__ uint32_t table_row(const AttnParams &p, const TableWindow &tw, int grp_clamped, int c) {
    const int blk = __shfl(tw.id, (grp_clamped >> p.bs_log2) - tw.first);
    return ((uint32_t) blk << p.bs_log2) | (uint32_t) (c & ((1 << p.bs_log2) - 1));
}

// Byte offset of pool row `row`.  The host admits only pools whose cell
// indices and row lengths fit in 32 bits (iian_pa_attention), so this is one
// 32x32 -> 64-bit multiply (v_mad_u64_u32) instead of a 64x64 product.
__device__ __forceinline__ uint64_t pool_off(uint32_t row, int64_t row_bytes) {
    return (uint64_t) row * (uint32_t) row_bytes;
}

// Orders this wave's LDS accesses before every wave's accesses after it
// (lgkmcnt(0), then s_barrier when the workgroup has several waves).  Unlike
// __syncthreads it does not wait for the global loads in flight, which are the
// prefetch of later tiles.
template <int NW>
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); vmcnt, expcnt not waited
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if constexpr (NW > 1) __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The cells base + off, off in [0, span), that a query row at position prow
// sees, as one range of offsets [lo, lo + width).  Cell c is visible when
// c < L, c <= prow under the causal mask, and prow - c < n_swa under a
// sliding window (paged_attn.cpp:124); each condition is a bound on off.  Per cell the test is then one subtract and one unsigned
// compare, with no branch (cell_visible).
struct CellWindow {
    int lo;
    uint32_t width;
};
__device__ __forceinline__ CellWindow cell_window(int base, int span, int L, int prow, int causal, int n_swa) {
    int hi = min(span, L - base);
    if (causal) hi = min(hi, prow + 1 - base);
    const int lo = n_swa > 0 ? max(0, prow - n_swa + 1 - base) : 0;
    return {lo, (uint32_t) max(hi - lo, 0)};
}
__device__ __forceinline__ bool cell_visible(const CellWindow &cw, int off) {
    return (uint32_t) (off - cw.lo) < cw.width;
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    const _Float16 ha = (_Float16) a, hb = (_Float16) b;
    return (uint32_t) __builtin_bit_cast(uint16_t, ha) | ((uint32_t) __builtin_bit_cast(uint16_t, hb) << 16);
}

// 4 int8 (ggml Q8_0 quants) -> 4 exact f16 (two packed pairs): bias to
// unsigned, v_perm each byte under 0x64 (the f16 1024 + u), subtract 1152.
__device__ __forceinline__ void i8x4_to_f16(uint32_t x, uint32_t &lo, uint32_t &hi) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const uint32_t u = x ^ 0x80808080u;                                      // q + 128
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);   // f16 {1024 + u0, 1024 + u1}
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);   // f16 {1024 + u2, 1024 + u3}
    const f16x2_t bias = {(_Float16) 1152.0f, (_Float16) 1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, a) - bias);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, b) - bias);
}

// 8 floats x*s -> an f16 pair (hi, lo) with hi = f16(x*s), lo = f16(x*s - hi),
// so hi + lo carries x*s to ~2^-22 relative.  A single f16 q has 2^-11
// relative error, and a score error of |s|*2^-11 becomes visible once the
// softmax is peaked (|s| of tens); the extra MFMA per k-step over lo keeps the
// scores at the reference's f32 q precision.
//
// hi and the difference pass through empty asm so that the compiler cannot
// fold "x*s - hi" into a v_fma_mix*_f16 with a negated operand: on MI355X
// (ROCm 7.2 hipcc) that form came out as hi - x*s, i.e. hi + lo = 2hi - x,
// twice the error of a plain f16 q (found by the peaked-softmax parity tests).
__device__ __forceinline__ void split_f16x8(const float4 &a, const float4 &b, float s, f16x8 &hi, f16x8 &lo) {
    const float x[8] = {a.x * s, a.y * s, a.z * s, a.w * s, b.x * s, b.y * s, b.z * s, b.w * s};
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float h = (float) (_Float16) x[e];
        asm volatile("" : "+v"(h));
        float d = x[e] - h;
        asm volatile("" : "+v"(d));
        hi[e] = (_Float16) h;
        lo[e] = (_Float16) d;
    }
}

}  // namespace iian_pa

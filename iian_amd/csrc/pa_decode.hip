// pa_decode.hip - stream-K paged decode / spec-verify attention for gfx950 (wave64, MFMA).
//
// The grid is a fixed number of single-wave workgroups; wave w takes an equal
// range of the call's (sequence, kv head, 32-cell tile) line (for_each_piece,
// pa_common.h), so ragged contexts leave no tail of idle CUs.  Within a
// piece the wave owns every query row of its sequence that maps to the kv
// head: row r = j*gqa + g for query token j and head g of the GQA group (so
// the group shares each K/V load), up to 16*NRT rows.  It walks its piece's cells in 32-cell tiles straight from the block
// table (no gather):
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
// The piece's block-table entries are read once into a register (lane i holds
// logical block first+i) and handed out with lane shuffles, so a tile's loads
// never wait on a table read.  Loads are single-buffered and phase-pipelined:
// the next tile's K loads are issued as soon as this tile's QK^T MFMAs have
// consumed K, its V loads as soon as V has been transposed, so they overlap the
// softmax and PV work of this tile.
//
// Pieces of a segment cut by worker boundaries write unnormalised partials
// (O, m, l); pa_merge_kernel combines them with a log-sum-exp merge.  A segment
// that is one piece writes its output directly.
// Semantics follow paged_attn_impl (src/iian/paged_attn.cpp:90-146): masks
// (:124), softcap (:127), all-masked rows -> 0 (:132).
#include "pa_common.h"
#include "pa_launch.h"
#include "pa_decode_body.h"

namespace iian_pa {

// 1.5 waves per SIMD are launched at D <= 128 (kF16DecodeWaves in pa_abi.hip),
// within a register budget of two waves per SIMD up to D*NRT = 128 (a budget
// of one wave per SIMD measured slower).
// WR: iian_pa_write_attention (the pieces write the step's new K/V rows).
template <int D, int NRT, int HG = 1, bool WR = false>
__global__ __launch_bounds__(64, (D * NRT <= 128) ? 2 : 1) void pa_decode_f16_kernel(AttnParams p) {
    for_each_piece<false>(p, blockIdx.x, 0, [&](const SeqWindow &w, const Piece &pc) {
        decode_piece<D, NRT, false, false, HG, WR>(p, w, pc);
    });
}

// Log-sum-exp merge of the stream-K partials: one workgroup per (sequence, kv
// head), wave i merging rows i, i+4, ...: out = sum_j 2^(m_j - m) O_j /
// sum_j 2^(m_j - m) l_j over the segment's pieces j, m = max_j m_j.  A separate
// launch: the kernel boundary is what makes the partials written on other XCDs
// visible (their L2s are not coherent within a launch, and a device-scope
// fence per piece costs an L2 write-back).
template <int D>
__global__ __launch_bounds__(256) void pa_merge_kernel(AttnParams p) {
    constexpr int DL = (D + 63) / 64;   // dims per lane (head size 96: 2 dims on lanes 0..47)
    constexpr bool ALL = D % 64 == 0;   // every lane has dims
    // blockIdx.y: the kv head, or the head group of head_group kv heads
    // (rows r of a group's segment: row r % M of its head r / M)
    const int s = blockIdx.x, hg = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool grouped = p.rec_heads > 1;
    // the segment table entry and the query range in one round trip: the
    // exit test below reads all three without short-circuit, so the entry is
    // not loaded after a branch on the query count
    const int2 info = p.seg_info[grouped ? s : s * (p.Hkv / p.head_group) + hg];
    const int qa = p.qsl[s], qb = p.qsl[s + 1];
    const int q0 = min(max(qa, 0), p.T);
    const int nq = min(max(qb, q0), p.T) - q0;
    const int M = nq * p.gqa;
    if ((nq <= 0) | (M > p.decode_rows) | (info.y <= 1)) return;
    const int hr = grouped ? hg : 0;
    const int rec0 = info.x, ns = info.y;
    const bool dl_live = ALL || lane * DL < D;
    for (int r = wave; r < M * p.head_group; r += 4) {
        const int hl = r / M, rh = r - hl * M;
        const int t = q0 + rh / p.gqa, h = (hg * p.head_group + hl) * p.gqa + rh % p.gqa;
        // the first 8 partial O rows are loaded together with the (m, l) of
        // pieces lane, lane + 64, ...; the first (m, l) chunk stays in registers
        float v0[8][DL];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float *op = rec_o(p, rec0 + min(u, ns - 1), hr, r, D) + lane * DL;
#pragma unroll
            for (int i = 0; i < DL; i++) v0[u][i] = dl_live ? op[i] : 0.f;
        }
        float2 ml0 = make_float2(-INFINITY, 0.f);
        if (lane < ns) ml0 = *(const float2 *) rec_ml(p, rec0 + lane, hr, r);
        float mx = ml0.x;
        for (int j = lane + 64; j < ns; j += 64) mx = fmaxf(mx, rec_ml(p, rec0 + j, hr, r)[0]);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        float acc[DL];
#pragma unroll
        for (int i = 0; i < DL; i++) acc[i] = 0.f;
        float lpart = 0.f;
        if (mx != -INFINITY) {
            for (int c0 = 0; c0 < ns; c0 += 64) {
                const int nc = min(64, ns - c0);
                const float2 ml = c0 == 0 ? ml0 : (lane < nc ? *(const float2 *) rec_ml(p, rec0 + c0 + lane, hr, r)
                                                             : make_float2(-INFINITY, 0.f));
                const float wl = lane < nc ? __builtin_amdgcn_exp2f(ml.x - mx) : 0.f;   // 0 for an empty piece
                lpart += wl * ml.y;
                // partial O rows in batches of 8, all loads of a batch issued before use
                for (int j0 = 0; j0 < nc; j0 += 8) {
                    float v[8][DL];
                    if (c0 == 0 && j0 == 0) {
#pragma unroll
                        for (int u = 0; u < 8; u++)
#pragma unroll
                            for (int i = 0; i < DL; i++) v[u][i] = v0[u][i];
                    } else {
#pragma unroll
                        for (int u = 0; u < 8; u++) {
                            const float *op = rec_o(p, rec0 + c0 + min(j0 + u, nc - 1), hr, r, D) + lane * DL;
#pragma unroll
                            for (int i = 0; i < DL; i++) v[u][i] = dl_live ? op[i] : 0.f;
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const float wgt = j0 + u < nc ? __shfl(wl, min(j0 + u, 63)) : 0.f;
#pragma unroll
                        for (int i = 0; i < DL; i++) acc[i] += wgt * v[u][i];
                    }
                }
            }
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) lpart += __shfl_xor(lpart, o);
        const float inv = lpart > 0.f ? 1.f / lpart : 0.f;
        float *out = p.out + ((int64_t) t * p.H + h) * D + lane * DL;
        if (dl_live)
#pragma unroll
            for (int i = 0; i < DL; i++) out[i] = acc[i] * inv;
    }
}

hipError_t launch_merge(const AttnParams &p, int head_dim, hipStream_t stream) {
    const dim3 grid(p.S, p.Hkv / p.head_group);
    switch (head_dim) {
        case 64: hipLaunchKernelGGL((pa_merge_kernel<64>), grid, dim3(256), 0, stream, p); break;
        case 96: hipLaunchKernelGGL((pa_merge_kernel<96>), grid, dim3(256), 0, stream, p); break;
        case 128: hipLaunchKernelGGL((pa_merge_kernel<128>), grid, dim3(256), 0, stream, p); break;
        case 256: hipLaunchKernelGGL((pa_merge_kernel<256>), grid, dim3(256), 0, stream, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Decode calls whose segments are short, or bounded by a sliding window
// (pa_abi.hip picks it): one workgroup of NW waves per (sequence, kv head)
// segment, wave w attending the segment's tiles [w*per, (w+1)*per),
// per = ceil(nt/NW).  The waves' records stay in LDS and the workgroup merges
// them after one barrier, so the call is one launch, with no records in HBM
// and no merge launch.  Its critical path is a chain of dependent memory round
// trips:
// - no window: one round trip carries the sequence's length and query range
//   and, beside them, the block-table entries from the wave's earliest
//   possible first tile (cell 32w) on.  Positions are not waited for: the
//   window is taken as [0, L) and every tile is masked by its rows' positions
//   (the tiles past a causal window contribute nothing).
// - sliding window: the window starts at the rows' smallest position minus
//   n_swa - 1, so a second round trip loads the positions and, beside them,
//   the table entries of the window that positions L - nq .. L - 1 (a decode
//   step's) would give; when the positions say otherwise the wave reloads its
//   entries.
// The stream-K kernel spreads a small call's few tiles over 1536 waves and
// then needs the merge launch and its round trips: at Qwen2.5-0.5B shapes its
// call takes 15.9 us (decode 8.1 + merge 5.4 us of kernel time) against 15.1
// us here, 15.5 against 12.8 us with the pool resident in the caches.  At
// Gemma3-12B's sliding-window layer (256 segments of 1024-cell windows, D =
// 256) the call takes 54.4-54.6 us here against 56.8-58.8 us (4 waves per
// segment; 3 waves measured the same, 2 waves 58.5 us).
template <int D, int NW, bool WR = false>
__global__ __launch_bounds__(64 * NW) void pa_decode_seg_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) float lrec[NW][16 * D + 32];
    const int s = blockIdx.x / p.Hkv, hk = blockIdx.x - s * p.Hkv;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const bool swa = p.n_swa > 0;
    // table entries clamped into the row (entries past the sequence's blocks
    // are never used)
    TableWindow tw;
    int32_t id = 0;
    if (!swa) {
        tw.first = (wave * kTile) >> p.bs_log2;
        id = p.bt[(int64_t) s * p.max_blocks + min(tw.first + lane, p.max_blocks - 1)];
    }
    SeqWindow w;
    w.L = max(p.seq_lens[s], 0);
    w.q0 = min(max(p.qsl[s], 0), p.T);
    w.nq = min(max(p.qsl[s + 1], w.q0), p.T) - w.q0;
    // a sequence with more query tokens than the caller's max_query_len may
    // have rows this launch does not cover (bit 2, as for_each_piece flags it)
    if (hk == 0 && threadIdx.x == 0 && w.nq > p.max_q && p.err) atomicOr(p.err, 4);
    if (w.nq <= 0 || w.nq * p.gqa > 16) return;   // workgroup-uniform
    if (!swa) {
        w.pmin = -1;        // no tile is taken as unmasked
        w.pmax = w.L - 1;   // (positions of padding rows, which are never written)
        w.c_lo = 0;
        w.c_hi = w.L;
    } else {
        const int lo_guess = max(0, w.L - w.nq - p.n_swa + 1) & ~(kTile - 1);
        const int per_guess = (max(1, (w.L - lo_guess + kTile - 1) / kTile) + NW - 1) / NW;
        tw.first = (lo_guess + wave * per_guess * kTile) >> p.bs_log2;
        id = p.bt[(int64_t) s * p.max_blocks + min(tw.first + lane, p.max_blocks - 1)];
        // the window of the rows' positions, as seq_window forms it
        int mn = INT32_MAX, mx = INT32_MIN;
        if (lane < w.nq) mn = mx = p.pos[w.q0 + lane];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            mn = min(mn, __shfl_xor(mn, o));
            mx = max(mx, __shfl_xor(mx, o));
        }
        w.pmin = __builtin_amdgcn_readfirstlane(mn);
        w.pmax = __builtin_amdgcn_readfirstlane(mx);
        int hi = w.L;
        if (p.causal) hi = min(hi, max(w.pmax + 1, 0));
        const int lo = max(0, w.pmin - p.n_swa + 1) & ~(kTile - 1);
        w.c_lo = lo;
        w.c_hi = max(hi, lo);
    }
    w.nt = max(1, (w.c_hi - w.c_lo + kTile - 1) / kTile);
    // as phys_block: a block past the table or a stale id is flagged, never
    // dereferenced
    const int nblk = (w.L + (1 << p.bs_log2) - 1) >> p.bs_log2;
    tw.id = id;
    if (tw.first + lane < nblk) {
        if (tw.first + lane >= p.max_blocks || (uint32_t) id >= (uint32_t) p.num_blocks) {
            if (p.err) atomicOr(p.err, 2);
            if ((uint32_t) id >= (uint32_t) p.num_blocks) tw.id = 0;
        }
    } else {
        tw.id = 0;
    }
    const int per = (w.nt + NW - 1) / NW;
    Piece pc;
    pc.s = s;
    pc.hk = hk;
    pc.t0 = wave * per;
    pc.t1 = min(w.nt, pc.t0 + per);
    pc.seg = s * p.Hkv + hk;
    pc.rec = pc.rec0 = 0;
    pc.pieces = (w.nt + per - 1) / per;
    if (pc.t0 < pc.t1) {
        // the loaded entries cover blocks first .. first+63: small block sizes
        // can leave the piece's first tile past them, and positions other than
        // the guessed ones can move it before them
        const int cb = w.c_lo + pc.t0 * kTile;
        const int c1 = min(cb + kTile - 1, w.L - 1);
        if ((cb >> p.bs_log2) < tw.first || (c1 >> p.bs_log2) - tw.first >= 64)
            table_load(p, s, cb >> p.bs_log2, w.L, tw);
        decode_piece<D, 1, false, true, 1, WR>(p, w, pc, &lrec[wave][0], &tw);
    }
    if (pc.pieces == 1) return;   // the one piece wrote the output
    __syncthreads();
    // log-sum-exp merge of the pieces' records, four dims per thread
    const int M = w.nq * p.gqa;
    for (int idx = threadIdx.x; idx < M * (D / 4); idx += 64 * NW) {
        const int r = idx / (D / 4), d = 4 * (idx % (D / 4));
        float mx = -INFINITY;
        for (int j = 0; j < pc.pieces; j++) mx = fmaxf(mx, lrec[j][16 * D + 2 * r]);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        float lsum = 0.f;
        if (mx != -INFINITY) {
            for (int j = 0; j < pc.pieces; j++) {
                const float wgt = __builtin_amdgcn_exp2f(lrec[j][16 * D + 2 * r] - mx);   // 0 for an empty piece
                lsum += wgt * lrec[j][16 * D + 2 * r + 1];
                const float4 v = *(const float4 *) &lrec[j][r * D + d];
                acc.x += wgt * v.x;
                acc.y += wgt * v.y;
                acc.z += wgt * v.z;
                acc.w += wgt * v.w;
            }
        }
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        const int t = w.q0 + r / p.gqa, h = hk * p.gqa + r % p.gqa;
        *(float4 *) (p.out + ((int64_t) t * p.H + h) * D + d) =
            make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    }
}

template <int D, int NRT, int HG = 1>
static hipError_t launch_decode_t(const AttnParams &p, hipStream_t stream) {
    const dim3 grid(p.sk_workers);
    if (p.k_new) hipLaunchKernelGGL((pa_decode_f16_kernel<D, NRT, HG, true>), grid, dim3(64), 0, stream, p);
    else hipLaunchKernelGGL((pa_decode_f16_kernel<D, NRT, HG>), grid, dim3(64), 0, stream, p);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : launch_merge(p, D, stream);
}

template <int D, int NW>
static void launch_seg(const AttnParams &p, dim3 grid, hipStream_t stream) {
    if (p.k_new) hipLaunchKernelGGL((pa_decode_seg_kernel<D, NW, true>), grid, dim3(64 * NW), 0, stream, p);
    else hipLaunchKernelGGL((pa_decode_seg_kernel<D, NW>), grid, dim3(64 * NW), 0, stream, p);
}

hipError_t launch_decode(const AttnParams &p, int head_dim, int kv_type, hipStream_t stream) {
    if (kv_type == 8) return launch_decode_q8(p, head_dim, stream);
    if (kv_type != 1) return hipErrorInvalidValue;
    if (p.head_group != 1 && head_dim != 96) return hipErrorInvalidValue;
    const int nrt = p.decode_rows > 16 ? 2 : 1;
    if (p.seg_waves > 0) {
        if (nrt != 1) return hipErrorInvalidValue;
        const dim3 grid((unsigned) ((int64_t) p.S * p.Hkv));
        if (head_dim == 64 && p.seg_waves == kSegWavesD64) launch_seg<64, kSegWavesD64>(p, grid, stream);
        else if (head_dim == 128 && p.seg_waves == kSegWavesD128) launch_seg<128, kSegWavesD128>(p, grid, stream);
        else if (head_dim == 256 && p.seg_waves == kSegWavesD256) launch_seg<256, kSegWavesD256>(p, grid, stream);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    switch (head_dim) {
        case 64: return nrt == 1 ? launch_decode_t<64, 1>(p, stream) : launch_decode_t<64, 2>(p, stream);
        case 96:
            if (p.head_group == 2) return nrt == 1 ? launch_decode_t<96, 1, 2>(p, stream) : hipErrorInvalidValue;
            return nrt == 1 ? launch_decode_t<96, 1>(p, stream) : launch_decode_t<96, 2>(p, stream);
        case 128: return nrt == 1 ? launch_decode_t<128, 1>(p, stream) : launch_decode_t<128, 2>(p, stream);
        case 256: return nrt == 1 ? launch_decode_t<256, 1>(p, stream) : launch_decode_t<256, 2>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iian_pa

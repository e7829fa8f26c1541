// pa_batch.hip - device-side batch metadata of one engine step.
//
// Engine::step builds its UBatch on the host by expanding every scheduled
// request's block table into absolute cells, one entry per context token
// (src/iian/engine.cpp:491-535; cell_of, include/iian/kv_cache.h:135-137):
// O(sum of context lengths) host work and transfer per step.  This kernel
// builds the arrays iian_pa_attention and iian_pa_kv_write read straight from
// the per-request state the scheduler already holds - the block ids of each
// request (KVRequestState::block_ids, kv_cache.h:93-97), its computed-token
// count and its new-token count - so the host uploads sum(blocks) + 3S
// integers instead of sum(context) cells.
//
// One workgroup per request s:
//   query_start_loc[s]  prefix sum of the new-token counts before s (each
//                       workgroup sums them itself: no second pass)
//   seq_lens[s]         num_computed + n_new
//   block_tables[s][b]  the request's block ids for the blocks its context
//                       uses, 0 after them (the padding PagedBatch uses)
//   pos[t], slots[t]    for its new tokens: pos = num_computed + i, slot =
//                       cell_of(pos) (engine.cpp:508-513)
#include "pa_common.h"
#include "pa_launch.h"

namespace iian_pa {

__global__ __launch_bounds__(256) void pa_build_batch_kernel(BatchParams p) {
    __shared__ int part[4];
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int acc = 0;
    for (int i = tid; i < s; i += 256) acc += max(p.n_new[i], 0);
    acc = wave_sum_i(acc);
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    const int q0 = part[0] + part[1] + part[2] + part[3];

    const int nc = p.num_computed[s], nn = p.n_new[s];
    const int off = p.block_off[s], nb = p.block_off[s + 1] - off;
    bool bad = nc < 0 || nn < 0 || nb < 0;
    const int L = max(nc, 0) + max(nn, 0);
    const int used = (L + p.block_size - 1) / p.block_size;
    // the request's blocks must cover its context and fit the table row
    bad |= used > nb || used > p.max_blocks;
    if (tid == 0) {
        p.seq_lens[s] = L;
        p.qsl[s] = q0;
        if (s == p.S - 1) {
            p.qsl[p.S] = q0 + max(nn, 0);
            bad |= q0 + max(nn, 0) != p.T;
        }
        if (bad && p.err) atomicOr(p.err, 8);
    }
    const int have = min(used, max(nb, 0));
    for (int b = tid; b < p.max_blocks; b += 256) {
        int32_t id = 0;
        if (b < have) {
            id = p.block_ids[off + b];
            if ((uint32_t) id >= (uint32_t) p.num_blocks && p.err) atomicOr(p.err, 2);
        }
        p.block_tables[(int64_t) s * p.max_blocks + b] = id;
    }
    for (int i = tid; i < nn; i += 256) {
        const int t = q0 + i;
        if (t >= p.T) {   // more new tokens than the caller's n_tokens (flagged above)
            if (p.err) atomicOr(p.err, 8);
            break;
        }
        const int ps = max(nc, 0) + i;
        const int b = ps / p.block_size;
        int64_t slot = -1;   // no block for this token: iian_pa_kv_write skips and flags slot -1
        if (b < max(nb, 0)) slot = (int64_t) p.block_ids[off + b] * p.block_size + (ps - b * p.block_size);
        else if (p.err) atomicOr(p.err, 1);
        p.pos[t] = ps;
        p.slots[t] = slot;
    }
    // Tokens past the last request's (the counts sum to less than n_tokens,
    // flagged above): slot -1, so a KV write of n_tokens rows skips them
    // instead of writing to whatever the buffers held.
    if (s == p.S - 1)
        for (int t = q0 + max(nn, 0) + tid; t < p.T; t += 256) {
            p.pos[t] = 0;
            p.slots[t] = -1;
        }
}

// Sliding-window block freeing (the reference's planned "free out-of-window
// blocks", docs/ROADMAP.md:33).  On a layer with window n_swa, a query at
// position q sees cells c > q - n_swa (src/iian/paged_attn.cpp:124), and the
// kernels start reading at that bound rounded down to a multiple of kTile.
// A sequence's later steps only have larger positions, so every block that
// ends at or before align_down(min_pos - n_swa + 1, kTile) is never read again
// by any kernel of this library: n_free[s] counts those leading blocks, and
// their table entries may be overwritten (with -1 here) and the blocks
// reused.  One wave per sequence.
__global__ __launch_bounds__(256) void pa_swa_free_kernel(const int32_t *__restrict__ qsl,
                                                          const int32_t *__restrict__ pos, int32_t S, int32_t T,
                                                          int32_t n_swa, int32_t block_size, int32_t *n_free,
                                                          int32_t *block_tables, int32_t max_blocks) {
    const int s = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (s >= S) return;
    const int q0 = min(max(qsl[s], 0), T), q1 = min(max(qsl[s + 1], q0), T);
    int mn = INT32_MAX;
    for (int t = q0 + lane; t < q1; t += 64) mn = min(mn, pos[t]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mn = min(mn, __shfl_xor(mn, o));
    int nf = 0;
    if (q1 > q0 && n_swa > 0) nf = (max(0, mn - n_swa + 1) & ~(kTile - 1)) / block_size;
    if (lane == 0) n_free[s] = nf;
    if (block_tables)
        for (int b = lane; b < min(nf, max_blocks); b += 64) block_tables[(int64_t) s * max_blocks + b] = -1;
}

hipError_t launch_swa_free(const int32_t *qsl, const int32_t *pos, int32_t S, int32_t T, int32_t n_swa,
                           int32_t block_size, int32_t *n_free, int32_t *block_tables, int32_t max_blocks,
                           hipStream_t stream) {
    hipLaunchKernelGGL(pa_swa_free_kernel, dim3((S + 3) / 4), dim3(256), 0, stream, qsl, pos, S, T, n_swa, block_size,
                       n_free, block_tables, max_blocks);
    return hipGetLastError();
}

hipError_t launch_build_batch(const BatchParams &p, hipStream_t stream) {
    hipLaunchKernelGGL(pa_build_batch_kernel, dim3(p.S), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace iian_pa

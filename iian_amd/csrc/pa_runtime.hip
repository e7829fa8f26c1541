// pa_runtime.hip - the engine-side runtime of the paged-attention path: the
// object an inference engine drives once per step and once per layer, so
// that paged attention runs with the KV cache on the GPU.
//
// In the reference the step's attention inputs are built on the host
// (Engine::step expands every request's block table into absolute cells,
// src/iian/engine.cpp:491-535) and every layer's build_attn emits two
// set_rows and the CPU paged op (src/iian/graph.cpp:314-337); on a GPU the
// reference cannot take that path at all (engine.cpp:187-188) and gathers K/V
// instead (graph.cpp:487-518).  This runtime owns the device buffers of one
// step (request state, block tables, seq_lens, query_start_loc, pos, slots,
// attention workspace, error word) and a double-buffered pinned staging area,
// allocated once at creation for the configured maxima:
//   begin_step  packs the scheduler's per-request block ids and token counts
//               into pinned memory, copies them to the device on the caller's
//               stream (asynchronously) and builds the step's arrays there
//               (iian_pa_build_batch)
//   layer       RoPE + the K/V write (iian_pa_rope_kv_write, or
//               iian_pa_kv_write_kv without RoPE) and paged attention
//               (iian_pa_attention) for one layer's pools
// Nothing is allocated after creation.  One runtime serves one stream at a
// time (its buffers are per step).
#include "../../include/iian_pa.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>

struct iian_pa_runtime {
    iian_pa_runtime_config cfg;
    int device = 0;
    // device buffers
    int32_t *d_req = nullptr;     // [block ids (max_total_blocks)][block_off (S+1)][num_computed (S)][n_new (S)]
    int32_t *d_bt = nullptr;      // [max_seqs][max_blocks_per_seq]
    int32_t *d_lens = nullptr;    // [max_seqs]
    int32_t *d_qsl = nullptr;     // [max_seqs + 1]
    int32_t *d_pos = nullptr;     // [max_tokens]
    int64_t *d_slots = nullptr;   // [max_tokens]
    int32_t *d_err = nullptr;     // [1]
    void *d_ws = nullptr;
    size_t ws_bytes = 0;
    // pinned staging of the request state, two areas used in turn; an area is
    // refilled only after the copy that read it has completed
    int32_t *h_stage[2] = {nullptr, nullptr};
    hipEvent_t staged[2] = {nullptr, nullptr};
    int next = 0;
    // the step in flight
    int32_t S = 0, T = 0, max_q = 0;
    bool in_step = false;
};

namespace {

size_t req_ints(const iian_pa_runtime_config &c) {
    return (size_t) c.max_total_blocks + (size_t) (c.max_seqs + 1) + 2 * (size_t) c.max_seqs;
}

void release(iian_pa_runtime *rt) {
    if (!rt) return;
    hipFree(rt->d_req);
    hipFree(rt->d_bt);
    hipFree(rt->d_lens);
    hipFree(rt->d_qsl);
    hipFree(rt->d_pos);
    hipFree(rt->d_slots);
    hipFree(rt->d_err);
    hipFree(rt->d_ws);
    for (int i = 0; i < 2; i++) {
        if (rt->h_stage[i]) hipHostFree(rt->h_stage[i]);
        if (rt->staged[i]) hipEventDestroy(rt->staged[i]);
    }
    delete rt;
}

}  // namespace

extern "C" {

int iian_pa_runtime_create(const iian_pa_runtime_config *cfg, iian_pa_runtime **out) {
    if (!cfg || !out) return IIAN_PA_ERR_NULL;
    *out = nullptr;
    const iian_pa_runtime_config &c = *cfg;
    if (c.max_seqs <= 0 || c.max_tokens <= 0 || c.max_blocks_per_seq <= 0 || c.max_total_blocks <= 0 ||
        c.n_head <= 0 || c.n_head_kv <= 0 || c.n_head % c.n_head_kv || c.block_size <= 0 || c.num_blocks <= 0)
        return IIAN_PA_ERR_ARG;
    if (!iian_pa_supported(c.type_k, c.type_v, c.head_dim, c.head_dim_v, 0.0f)) return IIAN_PA_ERR_UNSUPPORTED;
    iian_pa_runtime *rt = new (std::nothrow) iian_pa_runtime();
    if (!rt) return IIAN_PA_ERR_HIP;
    rt->cfg = c;
    if (hipGetDevice(&rt->device) != hipSuccess) {
        release(rt);
        return IIAN_PA_ERR_HIP;
    }
    rt->ws_bytes = iian_pa_workspace_size(c.max_tokens, c.max_seqs, c.n_head, c.n_head_kv, c.head_dim_v,
                                          c.max_blocks_per_seq, c.block_size);
    const size_t ri = req_ints(c);
    bool ok = rt->ws_bytes > 0 && hipMalloc(&rt->d_req, ri * sizeof(int32_t)) == hipSuccess &&
              hipMalloc(&rt->d_bt, (size_t) c.max_seqs * c.max_blocks_per_seq * sizeof(int32_t)) == hipSuccess &&
              hipMalloc(&rt->d_lens, (size_t) c.max_seqs * sizeof(int32_t)) == hipSuccess &&
              hipMalloc(&rt->d_qsl, (size_t) (c.max_seqs + 1) * sizeof(int32_t)) == hipSuccess &&
              hipMalloc(&rt->d_pos, (size_t) c.max_tokens * sizeof(int32_t)) == hipSuccess &&
              hipMalloc(&rt->d_slots, (size_t) c.max_tokens * sizeof(int64_t)) == hipSuccess &&
              hipMalloc(&rt->d_err, sizeof(int32_t)) == hipSuccess &&
              hipMalloc(&rt->d_ws, rt->ws_bytes) == hipSuccess && hipMemset(rt->d_err, 0, sizeof(int32_t)) == hipSuccess;
    for (int i = 0; ok && i < 2; i++)
        ok = hipHostMalloc((void **) &rt->h_stage[i], ri * sizeof(int32_t), hipHostMallocDefault) == hipSuccess &&
             hipEventCreateWithFlags(&rt->staged[i], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        release(rt);
        return IIAN_PA_ERR_HIP;
    }
    *out = rt;
    return IIAN_PA_OK;
}

void iian_pa_runtime_destroy(iian_pa_runtime *rt) {
    if (!rt) return;
    hipDeviceSynchronize();   // no copy or kernel of this runtime may still use its buffers
    release(rt);
}

int iian_pa_runtime_begin_step(iian_pa_runtime *rt, void *stream, const int32_t *const *block_ids,
                               const int32_t *n_blocks, const int32_t *num_computed, const int32_t *n_new,
                               int32_t n_seqs) {
    if (!rt) return IIAN_PA_ERR_NULL;
    rt->in_step = false;
    const iian_pa_runtime_config &c = rt->cfg;
    if (n_seqs <= 0 || n_seqs > c.max_seqs) return IIAN_PA_ERR_ARG;
    if (!block_ids || !n_blocks || !num_computed || !n_new) return IIAN_PA_ERR_NULL;
    // host-side checks of the request state (the engine's allocate_slots
    // guarantees them, include/iian/kv_cache.h:125-127)
    int64_t total_blocks = 0, T = 0;
    int32_t max_q = 0;
    for (int32_t s = 0; s < n_seqs; s++) {
        if (n_blocks[s] < 0 || num_computed[s] < 0 || n_new[s] < 0 || (n_blocks[s] > 0 && !block_ids[s]))
            return IIAN_PA_ERR_ARG;
        if ((int64_t) n_blocks[s] * c.block_size < (int64_t) num_computed[s] + n_new[s]) return IIAN_PA_ERR_ARG;
        total_blocks += n_blocks[s];
        T += n_new[s];
        max_q = std::max(max_q, n_new[s]);
    }
    if (total_blocks > c.max_total_blocks || T > c.max_tokens || T == 0) return IIAN_PA_ERR_ARG;
    for (int32_t s = 0; s < n_seqs; s++)
        if ((int64_t) num_computed[s] + n_new[s] > (int64_t) c.max_blocks_per_seq * c.block_size)
            return IIAN_PA_ERR_ARG;
    // pack into the staging area whose previous copy has completed
    const int a = rt->next;
    if (hipEventSynchronize(rt->staged[a]) != hipSuccess) return IIAN_PA_ERR_HIP;
    int32_t *h = rt->h_stage[a];
    int32_t *ids = h, *off = h + c.max_total_blocks, *nc = off + c.max_seqs + 1, *nn = nc + c.max_seqs;
    int64_t o = 0;
    off[0] = 0;
    for (int32_t s = 0; s < n_seqs; s++) {
        if (n_blocks[s]) std::memcpy(ids + o, block_ids[s], (size_t) n_blocks[s] * sizeof(int32_t));
        o += n_blocks[s];
        off[s + 1] = (int32_t) o;
    }
    std::memcpy(nc, num_computed, (size_t) n_seqs * sizeof(int32_t));
    std::memcpy(nn, n_new, (size_t) n_seqs * sizeof(int32_t));
    hipStream_t st = (hipStream_t) stream;
    if (hipMemcpyAsync(rt->d_req, h, req_ints(c) * sizeof(int32_t), hipMemcpyHostToDevice, st) != hipSuccess ||
        hipEventRecord(rt->staged[a], st) != hipSuccess)
        return IIAN_PA_ERR_HIP;
    rt->next = a ^ 1;
    const int32_t *d_ids = rt->d_req, *d_off = d_ids + c.max_total_blocks, *d_nc = d_off + c.max_seqs + 1,
                  *d_nn = d_nc + c.max_seqs;
    const int rc = iian_pa_build_batch(stream, d_ids, d_off, d_nc, d_nn, n_seqs, (int32_t) T, c.block_size,
                                       c.max_blocks_per_seq, c.num_blocks, rt->d_bt, rt->d_lens, rt->d_qsl, rt->d_pos,
                                       rt->d_slots, rt->d_err);
    if (rc) return rc;
    rt->S = n_seqs;
    rt->T = (int32_t) T;
    rt->max_q = max_q;
    rt->in_step = true;
    return IIAN_PA_OK;
}

int iian_pa_runtime_layer(iian_pa_runtime *rt, void *stream, const float *q, float *q_rot, const float *k_rows,
                          const float *v_rows, const iian_pa_rope_params *rope, void *k_pool, void *v_pool,
                          float scale, float softcap, int32_t causal, int32_t n_swa, float *out) {
    if (!rt) return IIAN_PA_ERR_NULL;
    if (!rt->in_step) return IIAN_PA_ERR_ARG;   // no begin_step (or it failed)
    const iian_pa_runtime_config &c = rt->cfg;
    const int64_t n_cells = (int64_t) c.num_blocks * c.block_size;
    int rc;
    const float *qa = q;
    if (rope) {
        if (!q_rot) return IIAN_PA_ERR_NULL;
        rc = iian_pa_rope_kv_write(stream, k_rows, v_rows, q, q_rot, rt->d_pos, rt->d_slots, rt->T, c.n_head,
                                   c.n_head_kv, c.head_dim, c.head_dim_v, rope, k_pool, v_pool, n_cells, c.type_k,
                                   c.type_v, rt->d_err);
        qa = q_rot;
    } else {
        rc = iian_pa_kv_write_kv(stream, k_rows, v_rows, rt->T, (int64_t) c.n_head_kv * c.head_dim,
                                 (int64_t) c.n_head_kv * c.head_dim_v, rt->d_slots, k_pool, v_pool, n_cells, c.type_k,
                                 c.type_v, rt->d_err);
    }
    if (rc) return rc;
    return iian_pa_attention(stream, qa, k_pool, v_pool, c.type_k, c.type_v, c.num_blocks, rt->d_bt,
                             c.max_blocks_per_seq, rt->d_lens, rt->d_qsl, rt->d_pos, rt->T, rt->S, rt->max_q,
                             c.n_head, c.n_head_kv, c.head_dim, c.head_dim_v, c.block_size, scale, softcap, causal,
                             n_swa, out, rt->d_ws, rt->ws_bytes, rt->d_err);
}

int iian_pa_runtime_errors(iian_pa_runtime *rt, void *stream, int32_t *host_err) {
    if (!rt || !host_err) return IIAN_PA_ERR_NULL;
    hipStream_t st = (hipStream_t) stream;
    if (hipMemcpyAsync(host_err, rt->d_err, sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess || hipMemsetAsync(rt->d_err, 0, sizeof(int32_t), st) != hipSuccess)
        return IIAN_PA_ERR_HIP;
    return IIAN_PA_OK;
}

}  // extern "C"

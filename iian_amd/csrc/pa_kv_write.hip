// pa_kv_write.hip - slot-mapped KV-cache write (set_rows) and Q8_0 dequantisation for gfx950.
//
// Semantics of ggml_set_rows as the reference uses it for the paged cache
// (src/iian/graph.cpp:314-322; CPU kernel ggml-cpu/ops.cpp:5221-5289):
// pool row slots[t] <- from_float(rows[t]).
//   F16  : IEEE binary16 round-to-nearest-even (v_cvt_f16_f32), as F16C's
//          _mm256_cvtps_ph(_MM_FROUND_TO_NEAREST_INT) (ggml-cpu.c:3480-3499).
//   Q8_0 : the x86 quantiser the reference engine runs on its host
//          (ggml-cpu/arch/x86/quants.c:302-398): d = amax/127.f (correctly
//          rounded divide), stored as f16(d); id = 127.f/amax; q = rint(x*id).
// Out-of-range slots are skipped (never written) and flagged in *err.
//
// Every write kernel takes a table of up to two (rows, pool, row length) jobs
// sharing one slot list, picked by blockIdx.y: the reference's two set_rows
// calls of a layer (K pool, then V pool, graph.cpp:319-320) run as one launch.
#include "pa_common.h"
#include "pa_launch.h"

namespace iian_pa {

struct WriteJob {
    const float *rows;
    void *pool;
    int64_t row_elems;
};
struct WriteJobs {
    WriteJob j[2];
};

__device__ __forceinline__ const WriteJob &pick(const WriteJobs &jobs) { return blockIdx.y ? jobs.j[1] : jobs.j[0]; }

// 8 elements per thread, 16-byte stores; requires row_elems % 8 == 0 and 16-byte aligned bases.
__global__ __launch_bounds__(256) void kv_write_f16_vec_kernel(WriteJobs jobs, int64_t n_rows,
                                                               const int64_t *__restrict__ slots, int64_t n_cells,
                                                               int32_t *err) {
    const WriteJob &jb = pick(jobs);
    const int64_t row_elems = jb.row_elems, per_row = row_elems >> 3;
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * per_row) return;
    const int64_t r = idx / per_row, c = idx - r * per_row;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (c == 0 && err) atomicOr(err, 1);
        return;
    }
    const float4 *src = (const float4 *) (jb.rows + r * row_elems + c * 8);
    const float4 a = src[0], b = src[1];
    const u32x4 v = {pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y), pack_f16x2(b.z, b.w)};
    *(u32x4 *) ((uint16_t *) jb.pool + slot * row_elems + c * 8) = v;
}

// Any alignment / row length: one element per thread.
__global__ __launch_bounds__(256) void kv_write_f16_scalar_kernel(WriteJobs jobs, int64_t n_rows,
                                                                  const int64_t *__restrict__ slots, int64_t n_cells,
                                                                  int32_t *err) {
    const WriteJob &jb = pick(jobs);
    const int64_t row_elems = jb.row_elems;
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * row_elems) return;
    const int64_t r = idx / row_elems, c = idx - r * row_elems;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (c == 0 && err) atomicOr(err, 1);
        return;
    }
    const _Float16 h = (_Float16) jb.rows[r * row_elems + c];
    ((uint16_t *) jb.pool)[slot * row_elems + c] = __builtin_bit_cast(uint16_t, h);
}

__global__ __launch_bounds__(256) void kv_write_f32_kernel(WriteJobs jobs, int64_t n_rows,
                                                           const int64_t *__restrict__ slots, int64_t n_cells,
                                                           int32_t *err) {
    const WriteJob &jb = pick(jobs);
    const int64_t row_elems = jb.row_elems;
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * row_elems) return;
    const int64_t r = idx / row_elems, c = idx - r * row_elems;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (c == 0 && err) atomicOr(err, 1);
        return;
    }
    ((float *) jb.pool)[slot * row_elems + c] = jb.rows[r * row_elems + c];
}

// One thread per 32-value Q8_0 block (34 bytes: f16 d, 32 x int8).
__global__ __launch_bounds__(256) void kv_write_q8_0_kernel(WriteJobs jobs, int64_t n_rows,
                                                            const int64_t *__restrict__ slots, int64_t n_cells,
                                                            int32_t *err) {
    const WriteJob &jb = pick(jobs);
    const int64_t row_elems = jb.row_elems, nb = row_elems >> 5;
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const int64_t r = idx / nb, b = idx - r * nb;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (b == 0 && err) atomicOr(err, 1);
        return;
    }
    const float *x = jb.rows + r * row_elems + b * 32;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = x[j];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.f;
    const float id = amax != 0.f ? 127.f / amax : 0.f;
    uint16_t *dst = (uint16_t *) ((uint8_t *) jb.pool + slot * (nb * 34) + b * 34);   // 2-byte aligned
    dst[0] = __builtin_bit_cast(uint16_t, (_Float16) d);
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
        const int q0 = min(127, max(-128, (int) __builtin_rintf(v[j] * id)));
        const int q1 = min(127, max(-128, (int) __builtin_rintf(v[j + 1] * id)));
        dst[1 + j / 2] = (uint16_t) ((q0 & 0xff) | ((q1 & 0xff) << 8));
    }
}

// ggml-quants.c:553-567: y = q * fp32(d).  One thread per value.
__global__ __launch_bounds__(256) void dequant_q8_0_kernel(const uint8_t *__restrict__ pool,
                                                           int64_t n_cells, const int64_t *__restrict__ rows_idx,
                                                           int64_t n_rows, int64_t row_elems, float *__restrict__ out) {
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * row_elems) return;
    const int64_t r = idx / row_elems, j = idx - r * row_elems;
    if (rows_idx[r] < 0 || rows_idx[r] >= n_cells) {
        out[idx] = 0.f;
        return;
    }
    const uint8_t *blk = pool + rows_idx[r] * ((row_elems >> 5) * 34) + (j >> 5) * 34;
    const float d = (float) __builtin_bit_cast(_Float16, *(const uint16_t *) blk);
    out[idx] = (float) (int8_t) blk[2 + (j & 31)] * d;
}

static inline unsigned nblocks(int64_t n) { return (unsigned) ((n + 255) / 256); }

// One launch for n_jobs (1 or 2) jobs of the same pool type over one slot list.
static hipError_t launch_jobs(const WriteJobs &jobs, int n_jobs, int64_t n_rows, const int64_t *slots,
                              int64_t n_cells, int type, int32_t *err, hipStream_t stream) {
    if (n_rows == 0) return hipSuccess;
    int64_t max_elems = 0;
    bool vec = true;
    for (int i = 0; i < n_jobs; i++) {
        const WriteJob &jb = jobs.j[i];
        max_elems = jb.row_elems > max_elems ? jb.row_elems : max_elems;
        vec = vec && (jb.row_elems % 8) == 0 && ((uintptr_t) jb.rows % 16) == 0 && ((uintptr_t) jb.pool % 16) == 0;
    }
    const dim3 block(256);
    if (type == 1) {
        if (vec)
            hipLaunchKernelGGL(kv_write_f16_vec_kernel, dim3(nblocks(n_rows * (max_elems / 8)), n_jobs), block, 0,
                               stream, jobs, n_rows, slots, n_cells, err);
        else
            hipLaunchKernelGGL(kv_write_f16_scalar_kernel, dim3(nblocks(n_rows * max_elems), n_jobs), block, 0,
                               stream, jobs, n_rows, slots, n_cells, err);
    } else if (type == 0) {
        hipLaunchKernelGGL(kv_write_f32_kernel, dim3(nblocks(n_rows * max_elems), n_jobs), block, 0, stream, jobs,
                           n_rows, slots, n_cells, err);
    } else if (type == 8) {
        hipLaunchKernelGGL(kv_write_q8_0_kernel, dim3(nblocks(n_rows * (max_elems / 32)), n_jobs), block, 0, stream,
                           jobs, n_rows, slots, n_cells, err);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_kv_write(const float *rows, int64_t n_rows, int64_t row_elems, const int64_t *slots, void *pool,
                           int64_t n_cells, int type, int32_t *err, hipStream_t stream) {
    WriteJobs jobs{};
    jobs.j[0] = {rows, pool, row_elems};
    return launch_jobs(jobs, 1, n_rows, slots, n_cells, type, err, stream);
}

hipError_t launch_kv_write_kv(const float *k_rows, const float *v_rows, int64_t n_rows, int64_t k_row_elems,
                              int64_t v_row_elems, const int64_t *slots, void *k_pool, void *v_pool, int64_t n_cells,
                              int type_k, int type_v, int32_t *err, hipStream_t stream) {
    WriteJobs jobs{};
    jobs.j[0] = {k_rows, k_pool, k_row_elems};
    jobs.j[1] = {v_rows, v_pool, v_row_elems};
    if (type_k == type_v) return launch_jobs(jobs, 2, n_rows, slots, n_cells, type_k, err, stream);
    // different pool types: one launch per pool
    WriteJobs vj{};
    vj.j[0] = jobs.j[1];
    const hipError_t e = launch_jobs(jobs, 1, n_rows, slots, n_cells, type_k, err, stream);
    return e != hipSuccess ? e : launch_jobs(vj, 1, n_rows, slots, n_cells, type_v, err, stream);
}

hipError_t launch_dequant_q8_0(const void *pool, int64_t n_cells, const int64_t *rows_idx, int64_t n_rows,
                               int64_t row_elems, float *out, hipStream_t stream) {
    if (n_rows == 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_q8_0_kernel, dim3(nblocks(n_rows * row_elems)), dim3(256), 0, stream,
                       (const uint8_t *) pool, n_cells, rows_idx, n_rows, row_elems, out);
    return hipGetLastError();
}

}  // namespace iian_pa

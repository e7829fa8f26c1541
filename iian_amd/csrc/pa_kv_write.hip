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
#include "pa_common.h"
#include "pa_launch.h"

namespace iian_pa {

// 8 elements per thread, 16-byte stores; requires row_elems % 8 == 0 and 16-byte aligned bases.
__global__ __launch_bounds__(256) void kv_write_f16_vec_kernel(const float *__restrict__ rows, int64_t n_rows,
                                                               int64_t row_elems, const int64_t *__restrict__ slots,
                                                               uint16_t *__restrict__ pool, int64_t n_cells,
                                                               int32_t *err) {
    const int64_t per_row = row_elems >> 3;
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * per_row) return;
    const int64_t r = idx / per_row, c = idx - r * per_row;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (c == 0 && err) atomicOr(err, 1);
        return;
    }
    const float4 *src = (const float4 *) (rows + r * row_elems + c * 8);
    const float4 a = src[0], b = src[1];
    const u32x4 v = {pack_f16x2(a.x, a.y), pack_f16x2(a.z, a.w), pack_f16x2(b.x, b.y), pack_f16x2(b.z, b.w)};
    *(u32x4 *) (pool + slot * row_elems + c * 8) = v;
}

// Any alignment / row length: one element per thread.
__global__ __launch_bounds__(256) void kv_write_f16_scalar_kernel(const float *__restrict__ rows, int64_t n_rows,
                                                                  int64_t row_elems, const int64_t *__restrict__ slots,
                                                                  uint16_t *__restrict__ pool, int64_t n_cells,
                                                                  int32_t *err) {
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * row_elems) return;
    const int64_t r = idx / row_elems, c = idx - r * row_elems;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (c == 0 && err) atomicOr(err, 1);
        return;
    }
    const _Float16 h = (_Float16) rows[r * row_elems + c];
    pool[slot * row_elems + c] = __builtin_bit_cast(uint16_t, h);
}

__global__ __launch_bounds__(256) void kv_write_f32_kernel(const float *__restrict__ rows, int64_t n_rows,
                                                           int64_t row_elems, const int64_t *__restrict__ slots,
                                                           float *__restrict__ pool, int64_t n_cells, int32_t *err) {
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * row_elems) return;
    const int64_t r = idx / row_elems, c = idx - r * row_elems;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (c == 0 && err) atomicOr(err, 1);
        return;
    }
    pool[slot * row_elems + c] = rows[r * row_elems + c];
}

// One thread per 32-value Q8_0 block (34 bytes: f16 d, 32 x int8).
__global__ __launch_bounds__(256) void kv_write_q8_0_kernel(const float *__restrict__ rows, int64_t n_rows,
                                                            int64_t row_elems, const int64_t *__restrict__ slots,
                                                            uint8_t *__restrict__ pool, int64_t n_cells,
                                                            int32_t *err) {
    const int64_t nb = row_elems >> 5;
    const int64_t idx = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const int64_t r = idx / nb, b = idx - r * nb;
    const int64_t slot = slots[r];
    if (slot < 0 || slot >= n_cells) {
        if (b == 0 && err) atomicOr(err, 1);
        return;
    }
    const float *x = rows + r * row_elems + b * 32;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = x[j];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.f;
    const float id = amax != 0.f ? 127.f / amax : 0.f;
    uint16_t *dst = (uint16_t *) (pool + slot * (nb * 34) + b * 34);   // 2-byte aligned
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

hipError_t launch_kv_write(const float *rows, int64_t n_rows, int64_t row_elems, const int64_t *slots, void *pool,
                           int64_t n_cells, int type, int32_t *err, hipStream_t stream) {
    if (n_rows == 0) return hipSuccess;
    if (type == 1) {
        const bool vec = (row_elems % 8) == 0 && ((uintptr_t) rows % 16) == 0 && ((uintptr_t) pool % 16) == 0;
        if (vec)
            hipLaunchKernelGGL(kv_write_f16_vec_kernel, dim3(nblocks(n_rows * (row_elems / 8))), dim3(256), 0, stream,
                               rows, n_rows, row_elems, slots, (uint16_t *) pool, n_cells, err);
        else
            hipLaunchKernelGGL(kv_write_f16_scalar_kernel, dim3(nblocks(n_rows * row_elems)), dim3(256), 0, stream,
                               rows, n_rows, row_elems, slots, (uint16_t *) pool, n_cells, err);
    } else if (type == 0) {
        hipLaunchKernelGGL(kv_write_f32_kernel, dim3(nblocks(n_rows * row_elems)), dim3(256), 0, stream, rows, n_rows,
                           row_elems, slots, (float *) pool, n_cells, err);
    } else if (type == 8) {
        hipLaunchKernelGGL(kv_write_q8_0_kernel, dim3(nblocks(n_rows * (row_elems / 32))), dim3(256), 0, stream,
                           rows, n_rows, row_elems, slots, (uint8_t *) pool, n_cells, err);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant_q8_0(const void *pool, int64_t n_cells, const int64_t *rows_idx, int64_t n_rows,
                               int64_t row_elems, float *out, hipStream_t stream) {
    if (n_rows == 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_q8_0_kernel, dim3(nblocks(n_rows * row_elems)), dim3(256), 0, stream,
                       (const uint8_t *) pool, n_cells, rows_idx, n_rows, row_elems, out);
    return hipGetLastError();
}

}  // namespace iian_pa

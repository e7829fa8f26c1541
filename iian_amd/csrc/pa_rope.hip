// pa_rope.hip - RoPE fused into the slot-mapped KV write (and, optionally, the
// same rotation of q) for gfx950.
//
// In the reference, build_rope (src/iian/graph.cpp:250-253) rotates K with
// ggml_rope_ext, and build_attn then writes the rotated rows into the pool
// with ggml_set_rows (graph.cpp:319-320): the rotated K makes a round trip
// through memory between the two ops, and q takes its own rope launch.  Here
// one launch per step rotates K and writes it straight to its slot, writes V,
// and rotates q into the attention's q buffer.
//
// One workgroup per token t:
//   1. the (cos, sin) cache of pos[t], one thread per pair, as
//      ggml_rope_cache_init + rope_yarn compute it (ggml-cpu/ops.cpp:5958-5990):
//      theta starts at the position and is multiplied by theta_scale once per
//      pair (the same chain of fp32 products), divided by the pair's freq
//      factor, interpolated by freq_scale, mixed by the YaRN ramp when
//      ext_factor != 0; cos and sin are the correctly rounded fp32 values of
//      the fp32 angle (evaluated in fp64), times the magnitude scale;
//   2. every head of K (and q) rotated in pairs (NORMAL: (2i, 2i+1); NEOX:
//      (i, i + n_dims/2); rotate_pairs, ggml-cpu/ops.cpp:6063-6080),
//      y0 = x0 c - x1 s, y1 = x0 s + x1 c, each product rounded (no fused
//      multiply-add, as the C source reads), the dims past n_dims copied;
//   3. the rotated K row and the V row converted into the pools at slots[t]
//      exactly as iian_pa_kv_write converts them (f16 round-to-nearest-even,
//      ggml's x86 Q8_0 quantiser, or f32).
#include "pa_common.h"
#include "pa_launch.h"

namespace iian_pa {

namespace {

constexpr int kRopeThreads = 256;

// One row of `elems` f32 values at src (LDS or global) into pool row `slot`.
template <int TY>
__device__ __forceinline__ void rope_store_row(const float *src, int elems, void *pool, int64_t slot) {
    const int tid = threadIdx.x;
    if constexpr (TY == 0) {
        float *dst = (float *) pool + slot * elems;
        for (int i = tid; i < elems; i += kRopeThreads) dst[i] = src[i];
    } else if constexpr (TY == 1) {
        uint32_t *dst = (uint32_t *) ((uint16_t *) pool + slot * elems);   // elems is even
        for (int i = tid; i < elems / 2; i += kRopeThreads) dst[i] = pack_f16x2(src[2 * i], src[2 * i + 1]);
    } else {
        // ggml's x86 quantize_row_q8_0 (ggml-cpu/arch/x86/quants.c:302-398),
        // one thread per 32-value block, as kv_write_q8_0_kernel
        const int nb = elems >> 5;
        for (int b = tid; b < nb; b += kRopeThreads) {
            const float *x = src + 32 * b;
            float amax = 0.f;
            for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
            const float d = amax / 127.f;
            const float id = amax != 0.f ? 127.f / amax : 0.f;
            uint16_t *dst = (uint16_t *) ((uint8_t *) pool + slot * (int64_t) (nb * 34) + b * 34);
            dst[0] = __builtin_bit_cast(uint16_t, (_Float16) d);
            for (int j = 0; j < 32; j += 2) {
                const int q0 = min(127, max(-128, (int) __builtin_rintf(x[j] * id)));
                const int q1 = min(127, max(-128, (int) __builtin_rintf(x[j + 1] * id)));
                dst[1 + j / 2] = (uint16_t) ((q0 & 0xff) | ((q1 & 0xff) << 8));
            }
        }
    }
}

__device__ __forceinline__ float rope_ramp(float low, float high, int i0) {
    const float y = (float) (i0 / 2) - low;
    const float r = y / fmaxf(0.001f, high - low);
    return 1.f - fminf(1.f, fmaxf(0.f, r));
}

}  // namespace

// Rotated pair (y0, y1) of (x0, x1) by (c, s), each product rounded.
__device__ __forceinline__ float2 rope_rotate(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c, b = x1 * s, e = x0 * s, f = x1 * c;
    return make_float2(a - b, e + f);
}

// Dynamic LDS: cache [n_dims] | rotated K row [Hkv*D] (only for a Q8_0 K pool).
template <int KT, int VT>
__global__ __launch_bounds__(kRopeThreads) void pa_rope_kv_write_kernel(RopeParams p) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float rope_lds[];
    float *cache = rope_lds;
    float *krow = rope_lds + p.n_dims;
    const int t = blockIdx.x, tid = threadIdx.x;
    const int half = p.n_dims >> 1;

    // 1. (cos, sin) of every pair at this token's position
    if (tid < half) {
        float theta = (float) p.pos[t];
        for (int j = 0; j < tid; j++) theta *= p.theta_scale;
        const int i0 = 2 * tid;
        const float ff = p.freq_factors ? p.freq_factors[tid] : 1.0f;
        const float theta_extrap = theta / ff;
        const float theta_interp = p.freq_scale * theta_extrap;
        float th = theta_interp;
        if (p.ext_factor != 0.0f) {
            const float ramp_mix = rope_ramp(p.corr0, p.corr1, i0) * p.ext_factor;
            th = theta_interp * (1.f - ramp_mix) + theta_extrap * ramp_mix;
        }
        cache[i0] = (float) cos((double) th) * p.mscale;
        cache[i0 + 1] = (float) sin((double) th) * p.mscale;
    }
    __syncthreads();

    // 2. rotate: pair i of head h, NORMAL (2i, 2i+1) or NEOX (i, i + n_dims/2)
    auto pair_index = [&](int i, int &e0, int &e1) {
        e0 = p.mode == 0 ? 2 * i : i;
        e1 = p.mode == 0 ? 2 * i + 1 : i + half;
    };
    const int64_t slot = p.slots[t];
    const bool slot_ok = slot >= 0 && slot < p.n_cells;
    if (!slot_ok && tid == 0 && p.err) atomicOr(p.err, 1);
    const int kd = p.Hkv * p.D;
    const float *kin = p.k_rows + (int64_t) t * kd;
    // a Q8_0 K row is quantised per 32-value block, so it is rotated into LDS
    // first; f16 and f32 rows go straight to the pool
    if (slot_ok) {
        if constexpr (KT == 8) {
            for (int i = tid; i < p.Hkv * half; i += kRopeThreads) {
                const int h = i / half, j = i - h * half;
                int e0, e1;
                pair_index(j, e0, e1);
                const float2 y = rope_rotate(kin[h * p.D + e0], kin[h * p.D + e1], cache[2 * j], cache[2 * j + 1]);
                krow[h * p.D + e0] = y.x;
                krow[h * p.D + e1] = y.y;
            }
            for (int i = tid; i < p.Hkv * (p.D - p.n_dims); i += kRopeThreads) {
                const int h = i / (p.D - p.n_dims), e = p.n_dims + (i - h * (p.D - p.n_dims));
                krow[h * p.D + e] = kin[h * p.D + e];
            }
            __syncthreads();
            rope_store_row<8>(krow, kd, p.k_pool, slot);
        } else {
            for (int i = tid; i < p.Hkv * half; i += kRopeThreads) {
                const int h = i / half, j = i - h * half;
                int e0, e1;
                pair_index(j, e0, e1);
                const float2 y = rope_rotate(kin[h * p.D + e0], kin[h * p.D + e1], cache[2 * j], cache[2 * j + 1]);
                const int64_t r0 = slot * kd + h * p.D;
                if constexpr (KT == 0) {
                    ((float *) p.k_pool)[r0 + e0] = y.x;
                    ((float *) p.k_pool)[r0 + e1] = y.y;
                } else {
                    ((_Float16 *) p.k_pool)[r0 + e0] = (_Float16) y.x;
                    ((_Float16 *) p.k_pool)[r0 + e1] = (_Float16) y.y;
                }
            }
            for (int i = tid; i < p.Hkv * (p.D - p.n_dims); i += kRopeThreads) {
                const int h = i / (p.D - p.n_dims), e = p.n_dims + (i - h * (p.D - p.n_dims));
                const int64_t r = slot * kd + h * p.D + e;
                if constexpr (KT == 0)
                    ((float *) p.k_pool)[r] = kin[h * p.D + e];
                else
                    ((_Float16 *) p.k_pool)[r] = (_Float16) kin[h * p.D + e];
            }
        }
        // 3. V: converted as it is
        rope_store_row<VT>(p.v_rows + (int64_t) t * p.Hkv * p.Dv, p.Hkv * p.Dv, p.v_pool, slot);
    }

    // q: rotated into q_out (may be q_in itself: each pair is read before it is written, by one thread)
    if (p.q_in) {
        const float *qin = p.q_in + (int64_t) t * p.H * p.D;
        float *qout = p.q_out + (int64_t) t * p.H * p.D;
        for (int i = tid; i < p.H * half; i += kRopeThreads) {
            const int h = i / half, j = i - h * half;
            int e0, e1;
            pair_index(j, e0, e1);
            const float2 y = rope_rotate(qin[h * p.D + e0], qin[h * p.D + e1], cache[2 * j], cache[2 * j + 1]);
            qout[h * p.D + e0] = y.x;
            qout[h * p.D + e1] = y.y;
        }
        if (qout != qin)
            for (int i = tid; i < p.H * (p.D - p.n_dims); i += kRopeThreads) {
                const int h = i / (p.D - p.n_dims), e = p.n_dims + (i - h * (p.D - p.n_dims));
                qout[h * p.D + e] = qin[h * p.D + e];
            }
    }
}

template <int KT, int VT>
static hipError_t launch_rope_t(const RopeParams &p, hipStream_t stream) {
    const size_t lds = ((size_t) p.n_dims + (KT == 8 ? (size_t) p.Hkv * p.D : 0)) * sizeof(float);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void *) pa_rope_kv_write_kernel<KT, VT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((pa_rope_kv_write_kernel<KT, VT>), dim3((unsigned) p.T), dim3(kRopeThreads), lds, stream, p);
    return hipGetLastError();
}

template <int KT>
static hipError_t launch_rope_k(const RopeParams &p, int type_v, hipStream_t stream) {
    switch (type_v) {
        case 0: return launch_rope_t<KT, 0>(p, stream);
        case 1: return launch_rope_t<KT, 1>(p, stream);
        case 8: return launch_rope_t<KT, 8>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rope_kv_write(const RopeParams &p, int type_k, int type_v, hipStream_t stream) {
    switch (type_k) {
        case 0: return launch_rope_k<0>(p, type_v, stream);
        case 1: return launch_rope_k<1>(p, type_v, stream);
        case 8: return launch_rope_k<8>(p, type_v, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iian_pa

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
// Work split.  A token's rows are its H q heads (when q is given), its Hkv K
// heads and its Hkv V heads.  A workgroup of 4 waves takes one token and a
// chunk of its rows, one row per wave at a time; the host sizes the chunks so
// a launch holds about 2048 workgroups (at the Llama-3-8B decode step 12
// chunks of 4 rows per token, 768 workgroups; at 2048 or more tokens one
// workgroup per token):
//   1. the workgroup's threads compute the token's (cos, sin) table, one pair
//      per thread, as ggml_rope_cache_init + rope_yarn compute it
//      (ggml-cpu/ops.cpp:5958-5990): theta starts at the position and is
//      multiplied by theta_scale once per pair (the same chain of fp32
//      products), divided by the pair's freq factor, interpolated by
//      freq_scale, mixed by the YaRN ramp when ext_factor != 0; cos and sin
//      are the correctly rounded fp32 values of the fp32 angle (evaluated in
//      fp64), times the magnitude scale.  Computing it once per workgroup
//      rather than per row keeps the fp64 work off the critical path (per row
//      it made a 256-head-dim prefill step 4x slower than its memory traffic);
//   2. q and K rows are rotated in pairs (NORMAL: (2i, 2i+1); NEOX:
//      (i, i + n_dims/2); rotate_pairs, ggml-cpu/ops.cpp:6063-6080),
//      y0 = x0 c - x1 s, y1 = x0 s + x1 c, each product rounded (no fused
//      multiply-add, as the C source reads), the dims past n_dims copied;
//   3. rotated K rows and V rows go into the pools at slots[t], converted
//      exactly as iian_pa_kv_write converts them (f16 round-to-nearest-even,
//      ggml's x86 Q8_0 quantiser, or f32).  A NORMAL pair is two adjacent
//      elements, so f16 rows are stored as packed pairs; a Q8_0 row is staged
//      in the wave's LDS slice and quantised 16 lanes per 32-value block.
#include "pa_common.h"
#include "pa_launch.h"

#include <algorithm>

namespace iian_pa {

namespace {

constexpr int kRopeWaves = 4;           // waves (head rows in flight) per workgroup
constexpr int kRopeMaxPairs = kRopeWaves * 64;   // n_dims / 2: one table entry per thread
constexpr int kRopeQ8MaxDim = 512;      // largest head row staged for a Q8_0 pool
constexpr int kRopeTargetWgs = 2048;    // workgroups a launch aims for

__device__ __forceinline__ float rope_ramp(float low, float high, int i0) {
    const float y = (float) (i0 / 2) - low;
    const float r = y / fmaxf(0.001f, high - low);
    return 1.f - fminf(1.f, fmaxf(0.f, r));
}

// (cos, sin) of pair j whose chained angle (position times theta_scale^j, one
// rounded product at a time) is theta.
__device__ __forceinline__ float2 rope_cs(const RopeParams &p, float theta, int j) {
#pragma clang fp contract(off)
    const float ff = p.freq_factors ? p.freq_factors[j] : 1.0f;
    const float theta_extrap = theta / ff;
    const float theta_interp = p.freq_scale * theta_extrap;
    float th = theta_interp;
    if (p.ext_factor != 0.0f) {
        const float ramp_mix = rope_ramp(p.corr0, p.corr1, 2 * j) * p.ext_factor;
        th = theta_interp * (1.f - ramp_mix) + theta_extrap * ramp_mix;
    }
    return make_float2((float) cos((double) th) * p.mscale, (float) sin((double) th) * p.mscale);
}

// ggml's x86 quantize_row_q8_0 (ggml-cpu/arch/x86/quants.c:302-398) of the
// wave's staged row x[0..n) (n a multiple of 32) into the Q8_0 blocks at dst:
// 16 lanes per 32-value block, two values per lane; the block's amax by xor
// shuffles inside the 16 lanes, d = amax/127, id = 127/amax, q = rint(x*id).
__device__ __forceinline__ void rope_store_q8_0(const float *x, int n, uint8_t *dst, int lane) {
    const int nb = n >> 5, g = lane >> 4, i = lane & 15;
    for (int b0 = 0; b0 < nb; b0 += 4) {
        const int b = b0 + g;
        const bool live = b < nb;
        const float2 v = live ? *(const float2 *) (x + 32 * b + 2 * i) : make_float2(0.f, 0.f);
        float amax = fmaxf(fabsf(v.x), fabsf(v.y));
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
        if (live) {
            const float d = amax / 127.f;
            const float id = amax != 0.f ? 127.f / amax : 0.f;
            const int q0 = min(127, max(-128, (int) __builtin_rintf(v.x * id)));
            const int q1 = min(127, max(-128, (int) __builtin_rintf(v.y * id)));
            uint16_t *blk = (uint16_t *) (dst + 34 * b);
            blk[1 + i] = (uint16_t) ((q0 & 0xff) | ((q1 & 0xff) << 8));
            if (i == 0) blk[0] = __builtin_bit_cast(uint16_t, (_Float16) d);
        }
    }
}

}  // namespace

// Rotated pair (y0, y1) of (x0, x1) by (c, s), each product rounded.
__device__ __forceinline__ float2 rope_rotate(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c, b = x1 * s, e = x0 * s, f = x1 * c;
    return make_float2(a - b, e + f);
}

// Wave-scope ordering of the wave's own LDS slice: its writes are complete
// and visible to its lanes before the reads that follow.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Token blockIdx.x, rows [blockIdx.y * rows_per_wg, +rows_per_wg) of its
// nq + 2 Hkv rows: q head r (r < nq), K head r - nq, V head r - nq - Hkv.
template <int KT, int VT>
__global__ __launch_bounds__(kRopeWaves * 64) void pa_rope_kv_write_kernel(RopeParams p, int nq, int rows_per_wg) {
#pragma clang fp contract(off)
    constexpr bool STAGE = KT == 8 || VT == 8;
    __shared__ float2 cs_tab[kRopeMaxPairs];
    __shared__ __attribute__((aligned(16))) float stage[STAGE ? kRopeWaves : 1][STAGE ? kRopeQ8MaxDim : 1];
    const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rpt = nq + 2 * p.Hkv;
    const int r0 = blockIdx.y * rows_per_wg, r1 = min(rpt, r0 + rows_per_wg);
    const int half = p.n_dims >> 1;
    const bool ne = p.mode != 0;   // NEOX pairs (i, i + n_dims/2)
    const int64_t slot = p.slots[t];
    const bool slot_ok = slot >= 0 && slot < p.n_cells;
    if (blockIdx.y == 0 && threadIdx.x == 0 && !slot_ok && p.err) atomicOr(p.err, 1);
    // the table is needed by q rows and by K rows whose slot is in the pool
    const bool rotates = r0 < nq || (slot_ok && r0 < nq + p.Hkv);
    if (rotates) {
        const int j = threadIdx.x;   // half <= kRopeMaxPairs = the workgroup's threads
        if (j < half) {
            float theta = (float) p.pos[t];
            for (int i = 0; i < j; i++) theta *= p.theta_scale;
            cs_tab[j] = rope_cs(p, theta, j);
        }
        __syncthreads();
    }
    for (int r = r0 + wave; r < r1; r += kRopeWaves) {
        const int kind = r < nq ? 0 : r < nq + p.Hkv ? 1 : 2;   // q, K, V
        const int h = kind == 0 ? r : kind == 1 ? r - nq : r - nq - p.Hkv;
        if (kind == 0 || (kind == 1 && slot_ok)) {
            // q or K: rotate
            const float *in = kind == 0 ? p.q_in + ((int64_t) t * p.H + h) * p.D
                                        : p.k_rows + ((int64_t) t * p.Hkv + h) * p.D;
            float *qo = p.q_out + ((int64_t) t * p.H + h) * p.D;
            const int64_t kbase = slot * ((int64_t) p.Hkv * p.D) + (int64_t) h * p.D;   // K element index in the pool
            for (int j = lane; j < half; j += 64) {
                const float2 cs = cs_tab[j];
                const int e0 = ne ? j : 2 * j, e1 = ne ? j + half : 2 * j + 1;
                float2 x;
                if (ne) {
                    x.x = in[e0];
                    x.y = in[e1];
                } else {
                    x = *(const float2 *) (in + e0);
                }
                const float2 y = rope_rotate(x.x, x.y, cs.x, cs.y);
                if (kind == 0) {
                    if (ne) {
                        qo[e0] = y.x;
                        qo[e1] = y.y;
                    } else {
                        *(float2 *) (qo + e0) = y;
                    }
                } else if constexpr (KT == 0) {
                    float *k = (float *) p.k_pool + kbase;
                    if (ne) {
                        k[e0] = y.x;
                        k[e1] = y.y;
                    } else {
                        *(float2 *) (k + e0) = y;
                    }
                } else if constexpr (KT == 1) {
                    _Float16 *k = (_Float16 *) p.k_pool + kbase;
                    if (ne) {
                        k[e0] = (_Float16) y.x;
                        k[e1] = (_Float16) y.y;
                    } else {
                        *(uint32_t *) (k + e0) = pack_f16x2(y.x, y.y);
                    }
                } else {
                    stage[wave][e0] = y.x;
                    stage[wave][e1] = y.y;
                }
            }
            // dims past n_dims are copied (q in place: already there)
            for (int e = p.n_dims + lane; e < p.D; e += 64) {
                const float v = in[e];
                if (kind == 0) {
                    if (qo != in) qo[e] = v;
                } else if constexpr (KT == 0) {
                    ((float *) p.k_pool)[kbase + e] = v;
                } else if constexpr (KT == 1) {
                    ((_Float16 *) p.k_pool)[kbase + e] = (_Float16) v;
                } else {
                    stage[wave][e] = v;
                }
            }
            if constexpr (KT == 8) {
                if (kind == 1) {
                    wave_lds_sync();
                    const int64_t rb = (int64_t) p.Hkv * p.D / 32 * 34;
                    rope_store_q8_0(stage[wave], p.D, (uint8_t *) p.k_pool + slot * rb + (int64_t) h * (p.D / 32) * 34,
                                    lane);
                    wave_lds_sync();   // the slice is rewritten by the wave's next row
                }
            }
        } else if (kind == 2 && slot_ok) {
            // V: converted as it is, two adjacent elements per lane
            const float *in = p.v_rows + ((int64_t) t * p.Hkv + h) * p.Dv;
            const int64_t vbase = slot * ((int64_t) p.Hkv * p.Dv) + (int64_t) h * p.Dv;
            for (int i = lane; 2 * i < p.Dv; i += 64) {
                const float2 x = *(const float2 *) (in + 2 * i);
                if constexpr (VT == 0)
                    *(float2 *) ((float *) p.v_pool + vbase + 2 * i) = x;
                else if constexpr (VT == 1)
                    *(uint32_t *) ((_Float16 *) p.v_pool + vbase + 2 * i) = pack_f16x2(x.x, x.y);
                else
                    *(float2 *) (&stage[wave][2 * i]) = x;
            }
            if constexpr (VT == 8) {
                wave_lds_sync();
                const int64_t rb = (int64_t) p.Hkv * p.Dv / 32 * 34;
                rope_store_q8_0(stage[wave], p.Dv, (uint8_t *) p.v_pool + slot * rb + (int64_t) h * (p.Dv / 32) * 34,
                                lane);
                wave_lds_sync();
            }
        }
    }
}

// Rows per workgroup: a multiple of the 4 waves, sized so that the launch
// holds about kRopeTargetWgs workgroups (one row per wave when the step has
// few tokens, a whole token per workgroup when it has thousands).
template <int KT, int VT>
static hipError_t launch_rope_t(const RopeParams &p, hipStream_t stream) {
    const int nq = p.q_in ? p.H : 0;
    const int64_t rpt = nq + 2 * (int64_t) p.Hkv;
    const int64_t per_wave_all = (rpt + kRopeWaves - 1) / kRopeWaves;
    const int64_t want = ((int64_t) p.T * rpt + (int64_t) kRopeWaves * kRopeTargetWgs - 1) /
                         ((int64_t) kRopeWaves * kRopeTargetWgs);
    const int64_t per_wave = std::max<int64_t>(1, std::min(per_wave_all, want));
    const int64_t rows_per_wg = per_wave * kRopeWaves;
    const int64_t chunks = (rpt + rows_per_wg - 1) / rows_per_wg;
    if (chunks > 65535 || rpt > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((pa_rope_kv_write_kernel<KT, VT>), dim3((unsigned) p.T, (unsigned) chunks),
                       dim3(kRopeWaves * 64), 0, stream, p, nq, (int) rows_per_wg);
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
    // a Q8_0 head row is staged whole and quantised in its own 32-value
    // blocks; the (cos, sin) table holds one pair per thread
    if ((type_k == 8 && (p.D % 32 || p.D > kRopeQ8MaxDim)) || (type_v == 8 && (p.Dv % 32 || p.Dv > kRopeQ8MaxDim)) ||
        p.n_dims / 2 > kRopeMaxPairs)
        return hipErrorInvalidValue;
    switch (type_k) {
        case 0: return launch_rope_k<0>(p, type_v, stream);
        case 1: return launch_rope_k<1>(p, type_v, stream);
        case 8: return launch_rope_k<8>(p, type_v, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace iian_pa

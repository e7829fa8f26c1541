// pa_mfma.h - MFMA 32x32x16 and LDS tile helpers shared by the gfx950 prefill kernels.
//
// MFMA 32x32x16 operand layouts (lane l, h = l/32): A[m][k] holds
// A[l%32][8h .. 8h+7]; B holds B[8h .. 8h+7][l%32]; the f32 result register r
// holds D[8(r/4) + 4h + r%4][l%32].
#pragma once

#include "pa_common.h"

namespace iian_pa {

typedef float f32x16 __attribute__((ext_vector_type(16)));


// LDS tile layouts.  Register-staged tiles (Q8_0 pools, D = 64) use padded
// rows: the QK^T A operand reads 16 consecutive K rows per 16 lanes, each 4
// banks after the last; a V transpose read covers 4 rows x 32 bytes per 16
// lanes, rows 16 banks apart so the two dim halves of a lane half never share
// a bank.  Tiles loaded straight into LDS (f16 pools at D >= 128) fill 1 KB
// per wave instruction, so their rows are unpadded and the 16-byte chunks of
// row r are XOR-permuted by swz(r) instead: 16 consecutive rows read at one
// logical chunk hit 16 different chunk slots, and the 4 rows of a transpose
// read (two chunks each, both dim halves) hit 16 different ones.
template <int D, bool DMA>
struct PrefillShape {
    // cells per tile: 64 (two independent 32-cell S^T halves) up to D = 128;
    // 32 at D = 256, where a second half's scores would not fit in registers
    static constexpr int PT = D <= 128 ? 64 : 32;
    static constexpr int NH = PT / 32;                         // 32-cell halves per tile
    static constexpr int KK = D / 16;                          // QK^T k-steps (16 dims each)
    static constexpr int NO = D / 32;                          // PV output tiles (32 dims each)
    static constexpr int KSTRIDE = DMA ? D * 2 : D * 2 + 16;
    // (a V transpose read takes 64 bytes of each of 4 rows per 32 lanes, so
    // register-staged rows sit 16 or 48 dwords apart: 192 bytes at D = 64 and
    // 96, 320 at D = 128)
    static constexpr int VSTRIDE = (DMA || D == 96) ? D * 2 : D * 2 + 64;
    static constexpr int KBYTES = PT * KSTRIDE;
    static constexpr int VBYTES = PT * VSTRIDE;
    static constexpr int CHUNKS = PT * (D / 8);                // 16-byte chunks per tile per tensor
};

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Byte offset in a tile of byte `b` of row r.
template <int D, bool DMA>
__device__ __forceinline__ int tile_off(int r, int b, int stride) {
    if constexpr (DMA) return r * stride + ((((b >> 4) ^ swz(r & 15)) << 4) | (b & 15));
    else return r * stride + b;
}

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Two transpose reads at LDS byte addresses a0, a1.  Callers that read
// several tiles from one lane base pass the base through opaque() first, so
// that the constant tile offsets become ds_read immediates instead of a VALU
// add per read (the compiler otherwise merges them into a scalar and adds
// that to the lane base before every read).
__device__ __forceinline__ f16x8 lds_tr_b16x8_at(uint32_t a0, uint32_t a1) {
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *) (uintptr_t) a0);
    const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *) (uintptr_t) a1);
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 c = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(f16x8, c);
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t) (uintptr_t) p; }

typedef __attribute__((address_space(3))) f16x8 lds_f16x8;
__device__ __forceinline__ f16x8 lds_read_f16x8(uint32_t a) { return *(const lds_f16x8 *) (uintptr_t) a; }

__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ f16x8 lds_tr_b16x8(const char *p0, const char *p1) {
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *) (uintptr_t) p0);
    const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *) (uintptr_t) p1);
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 c = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(f16x8, c);
}

// 16 bytes per lane from global memory straight into LDS: lane i's bytes land
// at LDS byte lds_off + 16i (global_load_lds_dwordx4, LDS base in m0, latched
// at issue).  Issued from inline assembly on purpose: the compiler treats its
// own LDS-load builtin as a write to all of LDS and waits for every one in
// flight before any later LDS read, which would serialise a double-buffered
// tile stream.  Callers order the loads themselves: s_waitcnt vmcnt(0) and a
// workgroup barrier before the tile is read, and a barrier between the last
// read of a buffer and the loads that refill it.
__device__ __forceinline__ void lds_load16(const void *gptr, uint32_t lds_off) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_off), "v"(gptr) : "m0");
}

// The same with a wave-uniform 64-bit base in SGPRs and the lane's 32-bit
// byte offset (the saddr form): the per-instruction address work is scalar.
__device__ __forceinline__ void lds_load16_s(const void *sbase, uint32_t voff, uint32_t lds_off) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_off), "v"(voff), "s"(sbase) : "m0");
}

__device__ __forceinline__ f32x16 mfma32(const f16x8 &a, const f16x8 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ---- The lo product of q in OCP E5M2 (bf8) ----
//
// An OCP E5M2 value is the top byte of the f16 encoding (sign, the same 5-bit
// exponent with bias 15, the top 2 mantissa bits), so the f16 K rows in LDS
// become bf8 operands with one v_perm per 4 values: rounded toward zero,
// relative error below 2^-2.  The lo half of q (lo = x - f16(x), at most
// 2^-11 |x|) only has to carry a few bits for the pair to hold q to ~2^-14;
// it is stored as bf8(lo * 2^kLo8Shift), rounded to nearest even, and the
// scaled MFMA applies 2^-kLo8Shift to it.  v_mfma_scale_f32_32x32x64_f8f6f4
// takes 64 k values per lane pair at twice the issue time of one
// v_mfma_f32_32x32x16_f16: the lo product of 64 dims costs 2 f16-MFMA slots
// instead of 4.  Byte b of a lane's 32-byte operand (either side) carries the
// same k index for A and B, so any consistent assignment of dims to bytes
// computes the dot product.
typedef int i32x8 __attribute__((ext_vector_type(8)));
constexpr int kLo8Shift = 12;

__device__ __forceinline__ f32x16 mfma32_bf8_lo(const i32x8 &a, const i32x8 &b, const f32x16 &c) {
    // A scale 2^0 (E8M0 127), B scale 2^-kLo8Shift
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 1, 0, 127, 0, 127 - kLo8Shift);
}

// The top bytes (bf8, truncated) of the 4 f16 values in dwords lo, hi.
__device__ __forceinline__ uint32_t f16x4_top_bytes(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x07050301u);
}

// bf8 of x, rounded to nearest even through f16, saturating at 57344.
__device__ __forceinline__ uint32_t bf8_rne(float x) {
    const uint32_t u = __builtin_bit_cast(uint16_t, (_Float16) x);
    uint32_t m = u & 0x7fffu;
    m = (m + 0x7fu + ((m >> 8) & 1u)) >> 8;
    return ((u >> 8) & 0x80u) | min(m, 0x7bu);
}

}  // namespace iian_pa

// khq_mfma_util.h -- device helpers shared by the matrix-core KHQ kernels
// (gfx950: 64-lane wavefronts, 16x16x32 / 16x16x16 f16 MFMA).
//
// MFMA operand layouts (lane l, li = l % 16, lg = l / 16):
//   16x16x32 f16: A lane holds A[li][8 lg .. 8 lg + 7], B lane holds
//                 B[8 lg .. 8 lg + 7][li], C lane holds C[4 lg .. 4 lg + 3][li];
//   16x16x16 f16: the same with 4 K values per lane (4 lg .. 4 lg + 3).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace khq {
namespace mu {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Orders this wavefront's LDS traffic (lanes exchange data through LDS).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cross-lane moves inside a 16-lane row (DPP, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// max / sum over the 16 lanes of a row: xor 1, xor 2 (quad_perm), then
// row_half_mirror and row_mirror fold the quads and the half rows.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}

// cos / sin of an fp32 angle (radians): exact reduction to [-1/2, 1/2]
// revolutions in fp64, then the hardware sine/cosine (revolution input).
__device__ __forceinline__ void sincos_rev(float th, float& c, float& s) {
    double r = (double)th * 0.15915494309189535;  // 1 / (2 pi)
    r -= rint(r);
    const float rf = (float)r;
    c = __builtin_amdgcn_cosf(rf);
    s = __builtin_amdgcn_sinf(rf);
}

__device__ __forceinline__ float fexp(float x) { return __expf(x); }

// hi + lo fp16 split of two floats (hi truncated, lo carries the rest).
__device__ __forceinline__ void split2(float x, float y, _Float16& xh, _Float16& yh,
                                       _Float16& xl, _Float16& yl) {
    const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x, y));
    const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(x - (float)hi[0], y - (float)hi[1]));
    xh = hi[0];
    yh = hi[1];
    xl = lo[0];
    yl = lo[1];
}

__device__ __forceinline__ void split(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// x + m * (float)h where h is the low / high fp16 half of a packed pair
// (v_fma_mix: the fp16 operand is widened exactly, one rounding).
__device__ __forceinline__ float mix_lo(uint32_t hp, float m, float x) {
    float d;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(hp), "v"(m), "v"(x));
    return d;
}
__device__ __forceinline__ float mix_hi(uint32_t hp, float m, float x) {
    float d;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(d) : "v"(hp), "v"(m), "v"(x));
    return d;
}
__device__ __forceinline__ uint32_t pk_rtz(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, y));
}
// Packed fp16 (x, y), round to nearest even (gfx950 v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pk_rne(float x, float y) {
    uint32_t d;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(d) : "v"(x), "v"(y));
    return d;
}
// Packed fp16 hi (truncated) and lo (remainder) parts of (x, y).
__device__ __forceinline__ void split_pk(float x, float y, uint32_t& hi, uint32_t& lo) {
    hi = pk_rtz(x, y);
    lo = pk_rtz(mix_lo(hi, -1.0f, x), mix_hi(hi, -1.0f, y));
}
// One of the two parts per lane: m = 0 gives hi, m = -1 gives lo.
__device__ __forceinline__ uint32_t part_pk(float x, float y, float m) {
    const uint32_t hi = pk_rtz(x, y);
    return pk_rtz(mix_lo(hi, m, x), mix_hi(hi, m, y));
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;
// Buffer resource over n_bytes at p: loads past the end return zeros.
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t n_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)n_bytes,
                                             0x00020000);
}

// Unnormalised FWHT-256 across a wavefront holding 4 consecutive dims per lane.
// Butterfly partner values: xor 1 / xor 2 by DPP quad_perm, xor 4 / 8 / 16
// by ds_swizzle (bit mode inside 32 lanes), xor 32 by a lane permute.
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
    if constexpr (M == 1) return dpp<0xB1>(v);
    else if constexpr (M == 2) return dpp<0x4E>(v);
    else if constexpr (M == 4 || M == 8 || M == 16)
        return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (M << 10)));
    else return __shfl_xor(v, 32, 64);
}
template <int M>
__device__ __forceinline__ void fwht_stage(float (&v)[4], int lane) {
    // lower lane: v + partner; upper lane: partner - v (fma with +-1 is exact)
    const float s = (lane & M) ? -1.0f : 1.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = fmaf(s, v[c], xor_lane<M>(v[c]));
}
__device__ __forceinline__ void fwht256(float (&v)[4], int lane) {
    float a = v[0], b = v[1];
    v[0] = a + b; v[1] = a - b;
    a = v[2]; b = v[3];
    v[2] = a + b; v[3] = a - b;
    a = v[0]; b = v[2];
    v[0] = a + b; v[2] = a - b;
    a = v[1]; b = v[3];
    v[1] = a + b; v[3] = a - b;
    fwht_stage<1>(v, lane);
    fwht_stage<2>(v, lane);
    fwht_stage<4>(v, lane);
    fwht_stage<8>(v, lane);
    fwht_stage<16>(v, lane);
    fwht_stage<32>(v, lane);
}

}  // namespace mu
}  // namespace khq

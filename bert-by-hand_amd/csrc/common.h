// Device-side helpers shared by the gfx950 kernels of the embedding engine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bbh {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;
constexpr int kHidden = 384;
constexpr int kHeads = 12;
constexpr int kHeadDim = 32;
constexpr int kFfn = 1536;
constexpr int kVocab = 30522;
constexpr int kMaxPos = 512;
constexpr size_t kLdsMax = 160 * 1024;  // LDS per workgroup on gfx950
constexpr int kTypes = 2;

// Lane exchanges without the LDS.  __shfl_xor compiles to ds_bpermute, an
// LDS operation with LDS latency (and queued behind the kernel's other LDS
// traffic); these use the VALU.  xor_*(v, f) returns f(v, v of lane l ^ d):
//  - d = 32, 16: v_permlane32_swap / v_permlane16_swap, which hand every lane
//    the low- and the high-half value; f(low, high) equals f(v, partner) bit
//    for bit for f = + and fmax (both commutative).
//  - d = 8: DPP row_ror:8 (within a 16-lane row, l -> l ^ 8).
//  - d = 4: DPP row_shl:4 (reads lane l + 4) or row_shr:4 (lane l - 4), by
//    bit 2 of the lane.
//  - d = 2, 1: DPP quad_perm [2,3,0,1] / [1,0,3,2].
// (Lane mappings checked on the device.)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int D, class F>
__device__ __forceinline__ float xor_op(float v, F f) {
  if constexpr (D == 32) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return f(__uint_as_float(s[0]), __uint_as_float(s[1]));
  } else if constexpr (D == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return f(__uint_as_float(s[0]), __uint_as_float(s[1]));
  } else if constexpr (D == 8) {
    return f(v, dpp<0x128>(v));
  } else if constexpr (D == 4) {
    const float up = dpp<0x104>(v), down = dpp<0x114>(v);
    return f(v, (threadIdx.x & 4) ? down : up);
  } else if constexpr (D == 2) {
    return f(v, dpp<0x4E>(v));
  } else {
    static_assert(D == 1, "xor distance");
    return f(v, dpp<0xB1>(v));
  }
}
struct AddOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// Sum / max over the 64 lanes of a wavefront (butterfly at distances 32, 16,
// ..., 1; every lane gets it).
template <class F>
__device__ __forceinline__ float wave_reduce(float v, F f) {
  v = xor_op<32>(v, f);
  v = xor_op<16>(v, f);
  v = xor_op<8>(v, f);
  v = xor_op<4>(v, f);
  v = xor_op<2>(v, f);
  return xor_op<1>(v, f);
}
__device__ inline float wave_sum(float v) { return wave_reduce(v, AddOp{}); }
__device__ inline float wave_max(float v) { return wave_reduce(v, MaxOp{}); }

// Reduction over the four 16-lane groups that share lane % 16 (the lanes that
// hold one row / column of a 16x16 MFMA tile).
__device__ inline float group4_sum(float v) { return xor_op<32>(xor_op<16>(v, AddOp{}), AddOp{}); }
__device__ inline float group4_max(float v) { return xor_op<32>(xor_op<16>(v, MaxOp{}), MaxOp{}); }

// v + the value of lane l ^ 32 (equal to v + __shfl_xor(v, 32) bit for bit).
__device__ inline float xor32_sum(float v) { return xor_op<32>(v, AddOp{}); }

// Exact GELU, x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2)), with the device
// library's erff (src/kernels/matmul.cu:27-28 uses the same definition).
__device__ inline float gelu_erf(float v) {
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
}

// The same function for GEMM epilogues, with no transcendental: Phi(x) =
// 1/2 + u P(u^2), u = x clamped to [-4.5, 4.5], P of degree 9 fitted to
// erf(u / sqrt 2) / (2 u) for least maximum |GELU error| (Lawson-weighted
// least squares).  Evaluated in fp32: |error| <= 1.1e-5 for |x| < 3, <= 7.6e-5
// for |x| < 6, <= 1.8e-4 to |x| = 14 (the clamp: x Phi(-4.5) = 3.4e-6 x), and
// <= 1e-5 relative near 0; against fp16 output rounding of up to 2.4e-4 |y|
// (|y| >= 0.5) that moves <= 2% of outputs with |x| < 2 by one fp16 step.
// 13 VALU operations (one med3, one mul, ten fma, one mul) where the rcp +
// exp form costs the VALU time of ~25: the epilogue of the K = 384 GEMMs runs
// on the same SIMD issue as their MFMAs.
__device__ inline float gelu_poly(float x) {
  const float u = __builtin_amdgcn_fmed3f(x, -4.5f, 4.5f);
  const float t = u * u;
  float p = -1.726400164e-12f;
  p = fmaf(p, t, 2.022508966e-10f);
  p = fmaf(p, t, -1.056738341e-08f);
  p = fmaf(p, t, 3.278985616e-07f);
  p = fmaf(p, t, -6.813811524e-06f);
  p = fmaf(p, t, 1.017347458e-04f);
  p = fmaf(p, t, -1.142718364e-03f);
  p = fmaf(p, t, 9.891781956e-03f);
  p = fmaf(p, t, -6.642068923e-02f);
  p = fmaf(p, t, 3.989246786e-01f);
  return x * fmaf(u, p, 0.5f);
}

// LayerNorm of one 384-wide row held by a wavefront: lane l holds columns
// 2l + 128j (j = 0, 1, 2) as v[2j], v[2j+1].  Two-pass mean and variance over
// the registers (src/kernels/layernorm.cu:32-49 reads the row three times);
// on return v holds (v - mean) * rstd.
__device__ __forceinline__ void ln_row384(float (&v)[6], float eps) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 6; ++e) s += v[e];
  const float mean = wave_sum(s) * (1.0f / kHidden);
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 6; ++e) {
    v[e] -= mean;
    q += v[e] * v[e];
  }
  const float rstd = rsqrtf(wave_sum(q) * (1.0f / kHidden) + eps);
#pragma unroll
  for (int e = 0; e < 6; ++e) v[e] *= rstd;
}

// gamma / beta of a lane's columns (layout of ln_row384), loaded before the
// row so that their latency overlaps the row's instead of following the
// reductions.
struct Affine384 {
  f16x2 g[3], b[3];
};
__device__ __forceinline__ Affine384 load_affine384(const f16* __restrict__ gamma,
                                                    const f16* __restrict__ beta, int lane) {
  Affine384 a;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    a.g[j] = *reinterpret_cast<const f16x2*>(gamma + 2 * lane + 128 * j);
    a.b[j] = *reinterpret_cast<const f16x2*>(beta + 2 * lane + 128 * j);
  }
  return a;
}

// fp16 of v * gamma[c] + beta[c] for the lane's column pair j (columns
// 2 lane + 128 j, +1), the expression every 384-wide LayerNorm row output
// goes through: an fp32 multiply-add, then the conversion.  The empty asm
// keeps the compiler from fusing the two into one v_fma_mix*_f16 (a single
// rounding) in some kernels and not in others.
__device__ __forceinline__ f16x2 affine384_pair(const float (&v)[6], const Affine384& a, int j) {
  float x0 = v[2 * j] * (float)a.g[j][0] + (float)a.b[j][0];
  float x1 = v[2 * j + 1] * (float)a.g[j][1] + (float)a.b[j][1];
  asm volatile("" : "+v"(x0), "+v"(x1));
  f16x2 o;
  o[0] = (f16)x0;
  o[1] = (f16)x1;
  return o;
}

// y[c] = v * gamma[c] + beta[c] for the lane's columns.
__device__ __forceinline__ void store_affine384(f16* __restrict__ y, const float (&v)[6],
                                                const Affine384& a, int lane) {
#pragma unroll
  for (int j = 0; j < 3; ++j)
    *reinterpret_cast<f16x2*>(y + 2 * lane + 128 * j) = affine384_pair(v, a, j);
}

// D(16x16, fp32) += A(16x32, fp16) . B(32x16, fp16) on the CDNA4 matrix core.
// Lane l supplies row (l % 16) of A and column (l % 16) of B, each as 8
// consecutive k values of k-group (l / 16); it receives D rows
// 4*(l/16) .. 4*(l/16)+3 of column (l % 16).
__device__ inline f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// D(32x32, fp32) += A(32x16, fp16) . B(16x32, fp16).  Lane l supplies row
// (l % 32) of A and column (l % 32) of B as the 8 k values 8*(l/32) .. +7; it
// receives D[8*(i/4) + 4*(l/32) + i%4][l % 32] in element i (checked on the
// device).  ~2.15 PFLOP/s sustained on MI355X against ~1.44 for the 16x16x32
// form.
__device__ inline f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

}  // namespace bbh

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
constexpr int kTypes = 2;

// Sum / max over the 64 lanes of a wavefront (butterfly, every lane gets it).
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Reduction over the four 16-lane groups that share lane % 16 (the lanes that
// hold one row / column of a 16x16 MFMA tile).
__device__ inline float group4_sum(float v) {
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

__device__ inline float group4_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

// Exact GELU, x * Phi(x) = 0.5 x (1 + erf(x / sqrt 2)), with the device
// library's erff (src/kernels/matmul.cu:27-28 uses the same definition).
__device__ inline float gelu_erf(float v) {
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
}

// The same function for GEMM epilogues, branch-free: with a = |x| and
// q = Phi(-a) = erfc(a / sqrt 2) / 2, x Phi(x) = x - a q for x >= 0 and
// -a q for x < 0, i.e. max(x, 0) - a q in both cases (one fma).  erfc(z) =
// t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2), t = 1 / (1 + p z):
// Abramowitz & Stegun, Handbook of Mathematical Functions (1964), eq. 7.1.26
// (after Hastings), |error in erfc| <= 1.5e-7, i.e. an absolute GELU error
// below 1e-7 |x| -- far under fp16 resolution.  The 1/2 and 1/sqrt 2 are
// folded into the constants; measured ~11% fewer VALU cycles than the
// sign-select form.
__device__ inline float gelu_as(float x) {
  const float a = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f * 0.70710678118654752440f, a, 1.0f));
  float p = fmaf(t, 0.5f * 1.061405429f, 0.5f * -1.453152027f);
  p = fmaf(t, p, 0.5f * 1.421413741f);
  p = fmaf(t, p, 0.5f * -0.284496736f);
  p = fmaf(t, p, 0.5f * 0.254829592f);
  // exp(-a^2 / 2) as exp2(a * (a * (-log2(e) / 2)))
  const float e = __builtin_amdgcn_exp2f(a * (a * (-0.5f * 1.4426950408889634f)));
  return fmaf(-a, t * p * e, fmaxf(x, 0.f));
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

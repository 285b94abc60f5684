// Linear layers of the encoder on the CDNA4 matrix cores.
//
// Every Linear in the path is C(M,N) = A(M,K) . W(N,K)^T with the torch
// (out, in) weight layout (reference: src/kernels/matmul.h:1-13), so both
// operands are K-contiguous.  The kernels compute the transposed tile
// D(n, m) = W . A^T with v_mfma_f32_16x16x32_f16: lane l then owns four
// consecutive output columns n of one row m and stores them as one 8-byte
// write.  fp16 operands, fp32 accumulation (the reference accumulates in
// fp16 on GeForce, src/kernels/matmul.cu:97-110; CDNA4 runs fp32 accumulate at
// full rate).
//
// Operand staging: a workgroup of 4 wavefronts owns a BM x BN output tile and
// walks K in BK-wide slices.  Each slice of A and W is loaded from global
// memory in 16-byte chunks into registers while the matrix cores work on the
// previous slice, then written to the other half of a double-buffered LDS
// area.  Inside LDS, chunk c of row r is stored at slot c ^ f(r) so the 16
// rows read by one MFMA operand fetch fall into distinct bank groups.
//
// Epilogues: bias (+ exact-erf GELU) as in src/kernels/matmul.cu:23-30, or
// bias + residual + LayerNorm over the full 384-wide row, which folds the
// reference's separate launch_layernorm(x, ..., residual) call
// (src/model/encoder.cu:47-50, 61-64; src/kernels/layernorm.cu:17-59) into the
// producing GEMM.

#include "kernels.h"

namespace bbh {
namespace {

constexpr int kThreads = 256;

template <int BK>
__device__ __forceinline__ int lds_off(int r, int c) {
  if constexpr (BK == 64)
    return r * 64 + ((c ^ (r & 7)) << 3);
  else
    return r * 32 + ((c ^ ((r >> 1) & 3)) << 3);
}

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int TM = BM / WM, TN = BN / WN;  // wave tile (rows m, cols n)
  static constexpr int FM = TM / 16, FN = TN / 16;  // 16x16 MFMA tiles per wave
  static constexpr int CPR = BK / 8;                // 16-byte chunks per row
  static constexpr int A_CH = BM * CPR, W_CH = BN * CPR;
  static constexpr int A_LD = (A_CH + kThreads - 1) / kThreads;
  static constexpr int W_LD = (W_CH + kThreads - 1) / kThreads;
  static constexpr int STAGE = (BM + BN) * BK;  // halves per pipeline stage
  static constexpr size_t LDS = 2 * STAGE * sizeof(f16);
  static_assert(WM * WN == 4, "four wavefronts per workgroup");
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be 16-aligned");
  static_assert(BK == 32 || BK == 64, "BK");
};

// K loop shared by all MFMA GEMMs.  On return acc[fm][fn] holds the fp32
// product tile: lane (r16 = l%16, g = l/16) has D rows n = n0 + wn*TN + fn*16 +
// 4g + i (i < 4) of column m = m0 + wm*TM + fm*16 + r16.  Rows of A past M are
// read clamped to row M-1 (valid memory, results discarded by the caller).
template <class T>
__device__ __forceinline__ void mainloop(const f16* __restrict__ A,
                                         const f16* __restrict__ W, int M, int K,
                                         int m0, int n0, f16* smem,
                                         f32x4 (&acc)[T::FM][T::FN]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / T::WN, wn = wave % T::WN;
  const int r16 = lane & 15, g = lane >> 4;

#pragma unroll
  for (int fm = 0; fm < T::FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < T::FN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};

  f16x8 ra[T::A_LD], rw[T::W_LD];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < T::A_LD; ++i) {
      const int c = tid + i * kThreads;
      if (T::A_CH % kThreads == 0 || c < T::A_CH) {
        const int row = c / T::CPR, ch = c % T::CPR;
        const int gm = min(m0 + row, M - 1);
        ra[i] = *reinterpret_cast<const f16x8*>(A + (size_t)gm * K + k0 + ch * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < T::W_LD; ++i) {
      const int c = tid + i * kThreads;
      if (T::W_CH % kThreads == 0 || c < T::W_CH) {
        const int row = c / T::CPR, ch = c % T::CPR;
        rw[i] = *reinterpret_cast<const f16x8*>(W + (size_t)(n0 + row) * K + k0 + ch * 8);
      }
    }
  };
  auto sstore = [&](int buf) {
    f16* sA = smem + buf * T::STAGE;
    f16* sW = sA + T::BM * T::BK;
#pragma unroll
    for (int i = 0; i < T::A_LD; ++i) {
      const int c = tid + i * kThreads;
      if (T::A_CH % kThreads == 0 || c < T::A_CH)
        *reinterpret_cast<f16x8*>(sA + lds_off<T::BK>(c / T::CPR, c % T::CPR)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < T::W_LD; ++i) {
      const int c = tid + i * kThreads;
      if (T::W_CH % kThreads == 0 || c < T::W_CH)
        *reinterpret_cast<f16x8*>(sW + lds_off<T::BK>(c / T::CPR, c % T::CPR)) = rw[i];
    }
  };

  const int KT = K / T::BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * T::BK);
    const f16* sA = smem + cur * T::STAGE;
    const f16* sW = sA + T::BM * T::BK;
#pragma unroll
    for (int s = 0; s < T::BK / 32; ++s) {
      f16x8 a[T::FM], w[T::FN];
#pragma unroll
      for (int fm = 0; fm < T::FM; ++fm)
        a[fm] = *reinterpret_cast<const f16x8*>(
            sA + lds_off<T::BK>(wm * T::TM + fm * 16 + r16, s * 4 + g));
#pragma unroll
      for (int fn = 0; fn < T::FN; ++fn)
        w[fn] = *reinterpret_cast<const f16x8*>(
            sW + lds_off<T::BK>(wn * T::TN + fn * 16 + r16, s * 4 + g));
#pragma unroll
      for (int fm = 0; fm < T::FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < T::FN; ++fn) acc[fm][fn] = mfma16(w[fn], a[fm], acc[fm][fn]);
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }
}

template <class T, bool kGelu>
__global__ __launch_bounds__(kThreads) void gemm_bias_kernel(
    const f16* __restrict__ A, const f16* __restrict__ W, const f16* __restrict__ bias,
    f16* __restrict__ C, int M, int N, int K) {
  HIP_DYNAMIC_SHARED(f16, smem);
  const int m0 = blockIdx.y * T::BM, n0 = blockIdx.x * T::BN;
  f32x4 acc[T::FM][T::FN];
  mainloop<T>(A, W, M, K, m0, n0, smem, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / T::WN, wn = wave % T::WN;
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int fm = 0; fm < T::FM; ++fm) {
    const int m = m0 + wm * T::TM + fm * 16 + r16;
    if (m >= M) continue;
#pragma unroll
    for (int fn = 0; fn < T::FN; ++fn) {
      const int n = n0 + wn * T::TN + fn * 16 + g * 4;
      f16x4 bv = bias ? *reinterpret_cast<const f16x4*>(bias + n) : f16x4{0, 0, 0, 0};
      f16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc[fm][fn][i] + (float)bv[i];
        if (kGelu) v = gelu_erf(v);
        o[i] = (f16)v;
      }
      *reinterpret_cast<f16x4*>(C + (size_t)m * N + n) = o;
    }
  }
}

// y = LN(A . W^T + bias + residual) over rows of exactly 384 columns.  The
// workgroup owns BM full rows; the four wavefronts split the 384 columns
// (96 each), and row statistics are combined through LDS.  Two-pass mean /
// variance over the register-resident row, as src/kernels/layernorm.cu:32-49.
template <class T>
__global__ __launch_bounds__(kThreads) void gemm_ln_kernel(
    const f16* __restrict__ A, const f16* __restrict__ W, const f16* __restrict__ bias,
    const f16* residual, const f16* __restrict__ gamma, const f16* __restrict__ beta,
    f16* y, int M, int K, float eps) {
  static_assert(T::BN == kHidden && T::WM == 1 && T::WN == 4, "row-owning tile");
  HIP_DYNAMIC_SHARED(f16, smem);
  const int m0 = blockIdx.x * T::BM;
  f32x4 acc[T::FM][T::FN];
  mainloop<T>(A, W, M, K, m0, 0, smem, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  float* red = reinterpret_cast<float*>(smem);  // [2][4][BM]; LDS is free after the K loop

#pragma unroll
  for (int fm = 0; fm < T::FM; ++fm) {
    const int mm = min(m0 + fm * 16 + r16, M - 1);
#pragma unroll
    for (int fn = 0; fn < T::FN; ++fn) {
      const int n = wave * T::TN + fn * 16 + g * 4;
      const f16x4 bv = *reinterpret_cast<const f16x4*>(bias + n);
      const f16x4 rv = *reinterpret_cast<const f16x4*>(residual + (size_t)mm * kHidden + n);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[fm][fn][i] += (float)bv[i] + (float)rv[i];
    }
  }
#pragma unroll
  for (int fm = 0; fm < T::FM; ++fm) {
    float s = 0.f;
#pragma unroll
    for (int fn = 0; fn < T::FN; ++fn)
#pragma unroll
      for (int i = 0; i < 4; ++i) s += acc[fm][fn][i];
    s = group4_sum(s);
    if (g == 0) red[wave * T::BM + fm * 16 + r16] = s;
  }
  __syncthreads();
  float mean[T::FM], rstd[T::FM];
#pragma unroll
  for (int fm = 0; fm < T::FM; ++fm) {
    const int row = fm * 16 + r16;
    mean[fm] = (red[row] + red[T::BM + row] + red[2 * T::BM + row] + red[3 * T::BM + row]) *
               (1.0f / kHidden);
    float q = 0.f;
#pragma unroll
    for (int fn = 0; fn < T::FN; ++fn)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float d = acc[fm][fn][i] - mean[fm];
        q += d * d;
      }
    q = group4_sum(q);
    if (g == 0) red[4 * T::BM + wave * T::BM + row] = q;
  }
  __syncthreads();
#pragma unroll
  for (int fm = 0; fm < T::FM; ++fm) {
    const int row = fm * 16 + r16;
    const float var = (red[4 * T::BM + row] + red[5 * T::BM + row] + red[6 * T::BM + row] +
                       red[7 * T::BM + row]) *
                      (1.0f / kHidden);
    rstd[fm] = rsqrtf(var + eps);
  }
#pragma unroll
  for (int fm = 0; fm < T::FM; ++fm) {
    const int m = m0 + fm * 16 + r16;
    if (m >= M) continue;
#pragma unroll
    for (int fn = 0; fn < T::FN; ++fn) {
      const int n = wave * T::TN + fn * 16 + g * 4;
      const f16x4 gv = *reinterpret_cast<const f16x4*>(gamma + n);
      const f16x4 bv = *reinterpret_cast<const f16x4*>(beta + n);
      f16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = (f16)((acc[fm][fn][i] - mean[fm]) * rstd[fm] * (float)gv[i] + (float)bv[i]);
      *reinterpret_cast<f16x4*>(y + (size_t)m * kHidden + n) = o;
    }
  }
}

// Any-shape fallback (the role of src/kernels/matmul.cu:34-59): 16x16 output
// tile per 256 threads, fp32 accumulate, operands staged through LDS.
__global__ __launch_bounds__(256) void gemm_generic_kernel(
    const f16* __restrict__ A, const f16* __restrict__ W, const f16* __restrict__ bias,
    f16* __restrict__ C, int M, int N, int K, int gelu) {
  __shared__ float As[16][17], Ws[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int mb = blockIdx.y * 16, nb = blockIdx.x * 16;
  float acc = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    const int k = k0 + tx;
    As[ty][tx] = (mb + ty < M && k < K) ? (float)A[(size_t)(mb + ty) * K + k] : 0.f;
    Ws[ty][tx] = (nb + ty < N && k < K) ? (float)W[(size_t)(nb + ty) * K + k] : 0.f;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) acc += As[ty][kk] * Ws[tx][kk];
    __syncthreads();
  }
  const int m = mb + ty, n = nb + tx;
  if (m < M && n < N) {
    float v = acc + (bias ? (float)bias[n] : 0.f);
    if (gelu) v = gelu_erf(v);
    C[(size_t)m * N + n] = (f16)v;
  }
}

template <class K>
hipError_t set_lds(K kernel, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

template <class T, bool kGelu>
hipError_t launch_bias(const f16* A, const f16* W, const f16* bias, f16* C, int M, int N,
                       int K, hipStream_t s) {
  static hipError_t attr = set_lds(gemm_bias_kernel<T, kGelu>, T::LDS);
  if (attr != hipSuccess) return attr;
  dim3 grid(N / T::BN, (M + T::BM - 1) / T::BM);
  hipLaunchKernelGGL((gemm_bias_kernel<T, kGelu>), grid, dim3(kThreads), T::LDS, s, A, W,
                     bias, C, M, N, K);
  return hipGetLastError();
}

using TileBig = Tile<128, 128, 64, 2, 2>;
using TileSmall = Tile<64, 64, 64, 2, 2>;
using TileLn = Tile<32, 384, 32, 1, 4>;

}  // namespace

bool gemm_mfma_ok(int N, int K) { return N % 64 == 0 && K % 64 == 0; }

hipError_t gemm(const f16* A, const f16* W, const f16* bias, f16* C, int M, int N, int K,
                Act act, hipStream_t s) {
  const bool gelu = act == Act::kGelu;
  const bool aligned = (((uintptr_t)A | (uintptr_t)W | (uintptr_t)C) & 15) == 0 &&
                       ((uintptr_t)bias & 7) == 0;
  if (!gemm_mfma_ok(N, K) || !aligned) {
    dim3 grid((N + 15) / 16, (M + 15) / 16);
    hipLaunchKernelGGL(gemm_generic_kernel, grid, dim3(256), 0, s, A, W, bias, C, M, N, K,
                       gelu ? 1 : 0);
    return hipGetLastError();
  }
  const bool big = (N % 128 == 0) && (size_t)M * N >= (size_t)256 * 128 * 128;
  if (big)
    return gelu ? launch_bias<TileBig, true>(A, W, bias, C, M, N, K, s)
                : launch_bias<TileBig, false>(A, W, bias, C, M, N, K, s);
  return gelu ? launch_bias<TileSmall, true>(A, W, bias, C, M, N, K, s)
              : launch_bias<TileSmall, false>(A, W, bias, C, M, N, K, s);
}

hipError_t gemm_residual_ln(const f16* A, const f16* W, const f16* bias,
                            const f16* residual, const f16* gamma, const f16* beta,
                            f16* y, int M, int K, float eps, hipStream_t s) {
  using T = TileLn;
  static hipError_t attr = set_lds(gemm_ln_kernel<T>, T::LDS);
  if (attr != hipSuccess) return attr;
  dim3 grid((M + T::BM - 1) / T::BM);
  hipLaunchKernelGGL((gemm_ln_kernel<T>), grid, dim3(kThreads), T::LDS, s, A, W, bias,
                     residual, gamma, beta, y, M, K, eps);
  return hipGetLastError();
}

}  // namespace bbh

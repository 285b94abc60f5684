// Memory-bound row kernels: LayerNorm, embedding gather (+ LayerNorm),
// masked mean pool and L2 normalisation.
//
// For 384-wide rows one wavefront owns a row: lane l holds columns
// 2l + 128j (j = 0, 1, 2) as three 4-byte half2 loads, so each load
// instruction of the wavefront covers 256 contiguous bytes.  The row stays in
// registers; mean and variance are two butterfly reductions over those
// registers (two-pass, as src/kernels/layernorm.cu:32-49, but one global read
// instead of three).

#include <type_traits>

#include "kernels.h"

namespace bbh {
namespace {

constexpr int kRowsPerBlock = 4;  // one row per wavefront, 256 threads

// y = LN(x [+ residual]) for D == 384 (src/kernels/layernorm.cu:17-59).
__global__ __launch_bounds__(256) void ln384_kernel(const f16* x, const f16* residual,
                                                    const f16* __restrict__ gamma,
                                                    const f16* __restrict__ beta, f16* y,
                                                    int M, float eps) {
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const size_t off = (size_t)row * kHidden;
  const Affine384 aff = load_affine384(gamma, beta, lane);
  float v[6];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int c = 2 * lane + 128 * j;
    const f16x2 a = *reinterpret_cast<const f16x2*>(x + off + c);
    v[2 * j] = (float)a[0];
    v[2 * j + 1] = (float)a[1];
    if (residual) {
      const f16x2 r = *reinterpret_cast<const f16x2*>(residual + off + c);
      v[2 * j] += (float)r[0];
      v[2 * j + 1] += (float)r[1];
    }
  }
  ln_row384(v, eps);
  store_affine384(y + off, v, aff, lane);
}

// Any D: three strided passes per wavefront-owned row, fp32 statistics.
__global__ __launch_bounds__(256) void ln_generic_kernel(const f16* x, const f16* residual,
                                                         const f16* __restrict__ gamma,
                                                         const f16* __restrict__ beta, f16* y,
                                                         int M, int D, float eps) {
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const size_t off = (size_t)row * D;
  auto val = [&](int i) {
    float v = (float)x[off + i];
    if (residual) v += (float)residual[off + i];
    return v;
  };
  float s = 0.f;
  for (int i = lane; i < D; i += 64) s += val(i);
  const float mean = wave_sum(s) / (float)D;
  float q = 0.f;
  for (int i = lane; i < D; i += 64) {
    const float d = val(i) - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)D + eps);
  for (int i = lane; i < D; i += 64)
    y[off + i] = (f16)((val(i) - mean) * rstd * (float)gamma[i] + (float)beta[i]);
}

__device__ __forceinline__ int clamp_id(int v, int n) { return v < 0 ? 0 : (v >= n ? n - 1 : v); }

// One wavefront's row: LN(word[id] + pos[p] + type[tt]), the sum kept in fp32.
__device__ __forceinline__ void embed_row(int id_raw, int tt_raw, int p, const f16* word,
                                          const f16* pos, const f16* type, const f16* gamma,
                                          const f16* beta, f16* dst, float eps, int lane) {
  const int id = clamp_id(id_raw, kVocab), tt = clamp_id(tt_raw, kTypes);
  const f16* wr = word + (size_t)id * kHidden;
  const f16* pr = pos + (size_t)p * kHidden;
  const f16* tr = type + (size_t)tt * kHidden;
  const Affine384 aff = load_affine384(gamma, beta, lane);
  float v[6];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int c = 2 * lane + 128 * j;
    const f16x2 a = *reinterpret_cast<const f16x2*>(wr + c);
    const f16x2 q = *reinterpret_cast<const f16x2*>(pr + c);
    const f16x2 t = *reinterpret_cast<const f16x2*>(tr + c);
    v[2 * j] = (float)a[0] + (float)q[0] + (float)t[0];
    v[2 * j + 1] = (float)a[1] + (float)q[1] + (float)t[1];
  }
  ln_row384(v, eps);
  store_affine384(dst, v, aff, lane);
}

// out[row] = LN(word[id] + pos[row % seq] + type[tt]) (src/model/forward.cu:28-31;
// gather as src/kernels/embedding.cu:20-30, sum kept in fp32 into the LN).
__global__ __launch_bounds__(256) void embedding_ln_kernel(
    const int32_t* __restrict__ ids, const int32_t* __restrict__ types,
    const f16* __restrict__ word, const f16* __restrict__ pos, const f16* __restrict__ type,
    const f16* __restrict__ gamma, const f16* __restrict__ beta, f16* __restrict__ out, int M,
    int seq, float eps) {
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  embed_row(ids[row], types[row], row % seq, word, pos, type, gamma, beta,
            out + (size_t)row * kHidden, eps, lane);
}

// The packed layout: workgroup s embeds sentence s's len tokens, wavefront w
// positions w, w + kPackedEmbWaves, ... (most sentences: one row per wave).
constexpr int kPackedEmbWaves = 8;
__global__ __launch_bounds__(64 * kPackedEmbWaves) void embedding_ln_packed_kernel(
    const int32_t* __restrict__ ids, const int32_t* __restrict__ types,
    const f16* __restrict__ word, const f16* __restrict__ pos, const f16* __restrict__ type,
    const f16* __restrict__ gamma, const f16* __restrict__ beta, f16* __restrict__ out,
    const PackedSentence* __restrict__ sents, float eps) {
  const PackedSentence sn = sents[blockIdx.x];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int p = wave; p < sn.len; p += kPackedEmbWaves)
    embed_row(ids[sn.tok + p], types[sn.tok + p], p, word, pos, type, gamma, beta,
              out + (size_t)(sn.row + p) * kHidden, eps, lane);
}

// Plain gather-sum, any hidden size (src/kernels/embedding.cu:8-31).
__global__ __launch_bounds__(256) void embedding_kernel(
    const int32_t* __restrict__ ids, const int32_t* __restrict__ types,
    const f16* __restrict__ word, const f16* __restrict__ pos, const f16* __restrict__ type,
    f16* __restrict__ out, int seq, int hidden, size_t total) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const size_t row = idx / hidden;
  const int c = idx % hidden;
  const int id = clamp_id(ids[row], kVocab), tt = clamp_id(types[row], kTypes);
  const int p = row % seq;
  out[idx] = (f16)((float)word[(size_t)id * hidden + c] + (float)pos[(size_t)p * hidden + c] +
                   (float)type[(size_t)tt * hidden + c]);
}

// One workgroup per sentence: the four wavefronts sum disjoint sets of tokens
// (positions w, w+4, ... in increasing order) of the masked mean, combine
// through LDS, then wave 0 divides by max(count, 1) (src/kernels/pooling.cu:
// 21-31) and scales by 1 / max(||x||, 1e-12) (src/kernels/normalize.cu:7,
// 29-30).  `valid(p)` says whether position p is counted and `row(p)` is its
// hidden row.  Each wavefront first lists its counted positions in LDS (one
// ballot per 64 of them), then sums their rows four at a time, so the row
// loads are issued together instead of one mask-dependent load at a time; the
// sum order is the same as one position after another.  `xform(a)` maps a
// loaded row (the lane's three column pairs) to the values that are summed.
struct RowAsIs {
  __device__ __forceinline__ void operator()(f16x2 (&)[3]) const {}
};
template <class Valid, class RowOf, class Xform = RowAsIs>
__device__ __forceinline__ void pool_normalize_body(int seq, Valid valid, RowOf row,
                                                    f16* __restrict__ dst, Xform xform = {}) {
  __shared__ float part[4][kHidden];
  __shared__ int cnt_part[4];
  __shared__ short plist[4][kMaxPos / 4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int n = 0;
  for (int i0 = 0; i0 < (seq + 3) / 4; i0 += kWave) {
    const int p = wave + 4 * (i0 + lane);
    const bool v = p < seq && valid(p);
    const uint64_t bal = __ballot(v);
    if (v) plist[wave][n + __popcll(bal & ((1ull << lane) - 1))] = (short)p;
    n += __popcll(bal);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's list is in LDS
  __builtin_amdgcn_wave_barrier();
  float acc[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto add_rows = [&](auto cnt_c, int k) {
    constexpr int U = decltype(cnt_c)::value;
    f16x2 a[U][3];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const f16* hr = row(plist[wave][k + u]);
#pragma unroll
      for (int j = 0; j < 3; ++j) a[u][j] = *reinterpret_cast<const f16x2*>(hr + 2 * lane + 128 * j);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xform(a[u]);
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        acc[2 * j] += (float)a[u][j][0];
        acc[2 * j + 1] += (float)a[u][j][1];
      }
    }
  };
  int k = 0;
  for (; k + 4 <= n; k += 4) add_rows(std::integral_constant<int, 4>{}, k);
  for (; k < n; ++k) add_rows(std::integral_constant<int, 1>{}, k);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    part[wave][2 * lane + 128 * j] = acc[2 * j];
    part[wave][2 * lane + 128 * j + 1] = acc[2 * j + 1];
  }
  if (lane == 0) cnt_part[wave] = n;
  __syncthreads();
  if (wave != 0) return;
  const int total = cnt_part[0] + cnt_part[1] + cnt_part[2] + cnt_part[3];
  const float inv_cnt = 1.0f / (float)(total > 0 ? total : 1);
  float v[6], ss = 0.f;
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int c = 2 * lane + 128 * j + e;
      v[2 * j + e] = (part[0][c] + part[1][c] + part[2][c] + part[3][c]) * inv_cnt;
      ss += v[2 * j + e] * v[2 * j + e];
    }
  const float inv = 1.0f / fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    f16x2 o;
    o[0] = (f16)(v[2 * j] * inv);
    o[1] = (f16)(v[2 * j + 1] * inv);
    *reinterpret_cast<f16x2*>(dst + 2 * lane + 128 * j) = o;
  }
}

__global__ __launch_bounds__(256) void pool_normalize_kernel(const f16* __restrict__ hidden,
                                                             const int32_t* __restrict__ mask,
                                                             f16* __restrict__ out, int seq) {
  const int b = blockIdx.x;
  const f16* hb = hidden + (size_t)b * seq * kHidden;
  const int32_t* mb = mask + (size_t)b * seq;
  pool_normalize_body(
      seq, [&](int p) { return mb[p] != 0; }, [&](int p) { return hb + (size_t)p * kHidden; },
      out + (size_t)b * kHidden);
}

// The last encoder layer's residual LayerNorm and the pool in one pass: the
// rows are read before their LayerNorm (y = FFN2 output + residual), each
// counted row is normalised as ln384 does it, rounded to fp16 the same way,
// and summed; so the embedding equals ln384 followed by pool_normalize, bit
// for bit, with one launch and one read of the rows fewer.  Only the pooled
// rows are normalised, and none is written back.
struct RowLayerNorm {
  Affine384 aff;
  float eps;
  __device__ __forceinline__ void operator()(f16x2 (&a)[3]) const {
    float v[6];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      v[2 * j] = (float)a[j][0];
      v[2 * j + 1] = (float)a[j][1];
    }
    ln_row384(v, eps);
#pragma unroll
    for (int j = 0; j < 3; ++j) a[j] = affine384_pair(v, aff, j);
  }
};

__global__ __launch_bounds__(256) void ln_pool_normalize_kernel(
    const f16* __restrict__ y, const int32_t* __restrict__ mask, const f16* __restrict__ gamma,
    const f16* __restrict__ beta, float eps, f16* __restrict__ out, int seq) {
  const int b = blockIdx.x;
  const f16* yb = y + (size_t)b * seq * kHidden;
  const int32_t* mb = mask + (size_t)b * seq;
  const RowLayerNorm ln{load_affine384(gamma, beta, threadIdx.x & 63), eps};
  pool_normalize_body(
      seq, [&](int p) { return mb[p] != 0; }, [&](int p) { return yb + (size_t)p * kHidden; },
      out + (size_t)b * kHidden, ln);
}

// Packed sentences: position p of sentence s is hidden row sents[s].row + p.
__global__ __launch_bounds__(256) void pool_normalize_packed_kernel(
    const f16* __restrict__ hidden, const PackedSentence* __restrict__ sents,
    f16* __restrict__ out) {
  const PackedSentence sn = sents[blockIdx.x];
  const f16* hb = hidden + (size_t)sn.row * kHidden;
  pool_normalize_body(
      sn.len, [&](int) { return true; }, [&](int p) { return hb + (size_t)p * kHidden; },
      out + (size_t)sn.out_row * kHidden);
}

// out[b, d] = masked mean over seq, any dim (src/kernels/pooling.cu:8-32).
__global__ __launch_bounds__(256) void mean_pool_kernel(const f16* __restrict__ hidden,
                                                        const int32_t* __restrict__ mask,
                                                        f16* __restrict__ out, int batch,
                                                        int seq, int dim) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= batch * dim) return;
  const int b = idx / dim, d = idx % dim;
  float acc = 0.f;
  int cnt = 0;
  for (int s = 0; s < seq; ++s) {
    const int m = mask[(size_t)b * seq + s];
    if (m) {
      ++cnt;
      acc += (float)hidden[((size_t)b * seq + s) * dim + d];
    }
  }
  out[idx] = (f16)(acc / (float)(cnt > 0 ? cnt : 1));
}

// Rows of x /= max(||row||, 1e-12), one workgroup per row
// (src/kernels/normalize.cu:10-33).
__global__ __launch_bounds__(256) void l2_normalize_kernel(f16* x, int n) {
  __shared__ float part[4];
  f16* r = x + (size_t)blockIdx.x * n;
  float s = 0.f;
  for (int i = threadIdx.x; i < n; i += 256) {
    const float v = (float)r[i];
    s += v * v;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  const float inv = 1.0f / fmaxf(sqrtf(part[0] + part[1] + part[2] + part[3]), 1e-12f);
  for (int i = threadIdx.x; i < n; i += 256) r[i] = (f16)((float)r[i] * inv);
}

// Exact GELU in place (src/kernels/gelu.h:5-9, gelu.cu): eight values per
// thread with 16-byte accesses; the tail, or a buffer not 16-byte aligned,
// one value per thread.
__global__ __launch_bounds__(256) void gelu8_kernel(f16* x, size_t n8) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  f16x8 v = reinterpret_cast<f16x8*>(x)[i];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (f16)gelu_erf((float)v[j]);
  reinterpret_cast<f16x8*>(x)[i] = v;
}

__global__ __launch_bounds__(256) void gelu1_kernel(f16* x, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) x[i] = (f16)gelu_erf((float)x[i]);
}

}  // namespace

hipError_t layernorm(const f16* x, const f16* residual, const f16* gamma, const f16* beta,
                     f16* y, int M, int D, float eps, hipStream_t s) {
  const dim3 grid((M + kRowsPerBlock - 1) / kRowsPerBlock);
  const bool aligned = (((uintptr_t)x | (uintptr_t)residual | (uintptr_t)gamma |
                         (uintptr_t)beta | (uintptr_t)y) & 3) == 0;
  if (D == kHidden && aligned)
    hipLaunchKernelGGL(ln384_kernel, grid, dim3(256), 0, s, x, residual, gamma, beta, y, M, eps);
  else
    hipLaunchKernelGGL(ln_generic_kernel, grid, dim3(256), 0, s, x, residual, gamma, beta, y, M,
                       D, eps);
  return hipGetLastError();
}

hipError_t embedding(const int32_t* ids, const int32_t* types, const f16* word, const f16* pos,
                     const f16* type, f16* out, int batch, int seq, int hidden,
                     hipStream_t s) {
  const size_t total = (size_t)batch * seq * hidden;
  hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     ids, types, word, pos, type, out, seq, hidden, total);
  return hipGetLastError();
}

hipError_t embedding_ln(const int32_t* ids, const int32_t* types, const f16* word,
                        const f16* pos, const f16* type, const f16* gamma, const f16* beta,
                        f16* out, int batch, int seq, float eps, hipStream_t s) {
  const int M = batch * seq;
  hipLaunchKernelGGL(embedding_ln_kernel, dim3((M + kRowsPerBlock - 1) / kRowsPerBlock),
                     dim3(256), 0, s, ids, types, word, pos, type, gamma, beta, out, M, seq,
                     eps);
  return hipGetLastError();
}

hipError_t mean_pool(const f16* hidden, const int32_t* mask, f16* out, int batch, int seq,
                     int dim, hipStream_t s) {
  hipLaunchKernelGGL(mean_pool_kernel, dim3((batch * dim + 255) / 256), dim3(256), 0, s, hidden,
                     mask, out, batch, seq, dim);
  return hipGetLastError();
}

hipError_t l2_normalize(f16* x, int n, int batch, hipStream_t s) {
  hipLaunchKernelGGL(l2_normalize_kernel, dim3(batch), dim3(256), 0, s, x, n);
  return hipGetLastError();
}

hipError_t gelu(f16* x, size_t n, hipStream_t s) {
  const size_t n8 = ((uintptr_t)x & 15) ? 0 : n / 8;
  if (n8)
    hipLaunchKernelGGL(gelu8_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, x, n8);
  const size_t rest = n - n8 * 8;
  if (rest)
    hipLaunchKernelGGL(gelu1_kernel, dim3((unsigned)((rest + 255) / 256)), dim3(256), 0, s,
                       x + n8 * 8, rest);
  return hipGetLastError();
}

hipError_t embedding_ln_packed(const int32_t* ids, const int32_t* types, const f16* word,
                               const f16* pos, const f16* type, const f16* gamma,
                               const f16* beta, f16* out, const PackedSentence* sents, int n,
                               float eps, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(embedding_ln_packed_kernel, dim3(n), dim3(64 * kPackedEmbWaves), 0, s, ids,
                     types, word, pos, type, gamma, beta, out, sents, eps);
  return hipGetLastError();
}

hipError_t pool_normalize_packed(const f16* hidden, const PackedSentence* sents, int n, f16* out,
                                 hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(pool_normalize_packed_kernel, dim3(n), dim3(256), 0, s, hidden, sents, out);
  return hipGetLastError();
}

hipError_t pool_normalize(const f16* hidden, const int32_t* mask, f16* out, int batch, int seq,
                          hipStream_t s) {
  hipLaunchKernelGGL(pool_normalize_kernel, dim3(batch), dim3(256), 0, s, hidden, mask, out,
                     seq);
  return hipGetLastError();
}

hipError_t ln_pool_normalize(const f16* y, const int32_t* mask, const f16* gamma,
                             const f16* beta, float eps, f16* out, int batch, int seq,
                             hipStream_t s) {
  hipLaunchKernelGGL(ln_pool_normalize_kernel, dim3(batch), dim3(256), 0, s, y, mask, gamma, beta,
                     eps, out, seq);
  return hipGetLastError();
}

}  // namespace bbh

// Masked multi-head self-attention for head_dim 32, read straight out of the
// fused QKV activations (row stride 3*384, Q | K | V column blocks,
// src/model/weights.h:38-54; strided reads as src/kernels/attention.cu:25-28,
// 74-75) and written straight into the merged (B*S, 384) layout
// (attention.cu:87-92).
//
// The reference materialises scores (B*12, S, S) in HBM, runs a separate
// masked softmax over them and a third kernel for P.V
// (src/model/encoder.cu:39-45).  Here one kernel does all three per
// (batch, head, 16-query tile) with an online softmax, so scores never leave
// the chip; at S = 512 the reference layout would be 1.6 GB per layer.
//
// Per wavefront: 16 queries.  Keys are staged through LDS in blocks of 64
// (K row-major, V transposed to [dim][key]); each 32-key chunk costs
//   2 x v_mfma_f32_16x16x32_f16 for S^T = K . Q^T  (all 32 head dims at once)
//   online-softmax update in fp32 (exp2, scale folded with log2 e)
//   2 x v_mfma_f32_16x16x32_f16 for O^T = V^T . P^T
// The S^T accumulator of lane l holds query l%16 and keys 4(l/16)+i; the K
// rows of the two S^T tiles are permuted so that lane l's eight scores are the
// contiguous keys 8(l/16)..8(l/16)+7, which are exactly the eight k-values
// lane l must feed as operand B of the P.V product.  P therefore goes from
// accumulator to MFMA operand without leaving the lane.
//
// Mask semantics follow src/kernels/softmax.cu:35-62: keys with mask 0 are
// dropped; a query whose keys are all masked gets a zero context.  Chunks of
// 32 keys that are entirely masked are skipped (their contribution is exactly
// zero).

#include "kernels.h"

namespace bbh {
namespace {

constexpr int KB = 64;        // keys staged per LDS block
constexpr int VT_LD = KB + 8;  // padded row of the transposed V tile

// Slot of 16-byte chunk c (of 4) in K-tile row j; conflict-free for the key
// pattern one S^T operand fetch touches (rows {0,1,2,3,8,9,10,11} + const).
__device__ __forceinline__ int k_off(int j, int c) {
  const int sw = ((j >> 1) & 1) | ((j >> 2) & 2);
  return j * 32 + ((c ^ sw) << 3);
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void attention_kernel(const f16* __restrict__ qkv,
                                                            const int32_t* __restrict__ mask,
                                                            f16* __restrict__ out, int seq,
                                                            int heads, float scale_log2) {
  __shared__ __attribute__((aligned(16))) f16 Ks[KB * 32];
  __shared__ __attribute__((aligned(16))) f16 Vt[32 * VT_LD];
  __shared__ float mb[KB];

  const int b = blockIdx.z, h = blockIdx.y;
  const int hid = heads * kHeadDim, ld = 3 * hid;
  const f16* base = qkv + (size_t)b * seq * ld;
  const int32_t* mrow_ptr = mask + (size_t)b * seq;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int q0 = (blockIdx.x * NW + wave) * 16;
  const bool active = q0 < seq;
  const int q = min(q0 + r16, seq - 1);

  const f16x8 qf = *reinterpret_cast<const f16x8*>(base + (size_t)q * ld + h * kHeadDim + g * 8);
  f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
  float mrun = -INFINITY, lsum = 0.f;

  for (int kb = 0; kb < seq; kb += KB) {
    __syncthreads();  // previous block's LDS reads are done
    for (int c = tid; c < KB * 4; c += 64 * NW) {
      const int j = c >> 2, ch = c & 3, key = kb + j;
      f16x8 kv = {0, 0, 0, 0, 0, 0, 0, 0}, vv = kv;
      if (key < seq) {
        const f16* row = base + (size_t)key * ld + h * kHeadDim + ch * 8;
        kv = *reinterpret_cast<const f16x8*>(row + hid);
        vv = *reinterpret_cast<const f16x8*>(row + 2 * hid);
      }
      *reinterpret_cast<f16x8*>(&Ks[k_off(j, ch)]) = kv;
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[(ch * 8 + e) * VT_LD + j] = vv[e];
    }
    for (int j = tid; j < KB; j += 64 * NW) {
      const int key = kb + j;
      mb[j] = (key < seq && mrow_ptr[key] != 0) ? 0.f : -INFINITY;
    }
    __syncthreads();
    if (!active) continue;

    const int kend = min(KB, seq - kb);
    for (int kc = 0; kc < kend; kc += 32) {
      float mk[8];
      bool any = false;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        mk[e] = mb[kc + 8 * g + e];
        any |= (mk[e] == 0.f);
      }
      if (!__any(any)) continue;

      // S^T tiles: operand-A row r16 of tile t is key kc + 8(r16/4) + 4t + r16%4.
      const int kr0 = kc + 8 * (r16 >> 2) + (r16 & 3);
      const f16x8 k0 = *reinterpret_cast<const f16x8*>(&Ks[k_off(kr0, g)]);
      const f16x8 k1 = *reinterpret_cast<const f16x8*>(&Ks[k_off(kr0 + 4, g)]);
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 s0 = mfma16(k0, qf, zero);  // keys kc+8g+i
      const f32x4 s1 = mfma16(k1, qf, zero);  // keys kc+8g+4+i

      float sv[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[i] = s0[i] * scale_log2 + mk[i];
        sv[4 + i] = s1[i] * scale_log2 + mk[4 + i];
      }
      float cmax = sv[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) cmax = fmaxf(cmax, sv[e]);
      cmax = group4_max(cmax);
      const float mnew = fmaxf(mrun, cmax);
      const float muse = (mnew == -INFINITY) ? 0.f : mnew;
      const float corr = exp2f(mrun - muse);
      f16x8 p;
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pe = exp2f(sv[e] - muse);
        ps += pe;
        p[e] = (f16)pe;
      }
      lsum = lsum * corr + ps;
      mrun = mnew;
      o0 *= corr;
      o1 *= corr;
      const f16x8 v0 = *reinterpret_cast<const f16x8*>(&Vt[r16 * VT_LD + kc + 8 * g]);
      const f16x8 v1 = *reinterpret_cast<const f16x8*>(&Vt[(16 + r16) * VT_LD + kc + 8 * g]);
      o0 = mfma16(v0, p, o0);  // dims 4g+i of query r16
      o1 = mfma16(v1, p, o1);  // dims 16+4g+i
    }
  }
  if (!active) return;
  const float lt = group4_sum(lsum);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  f16x4 w0, w1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w0[i] = (f16)(o0[i] * inv);
    w1[i] = (f16)(o1[i] * inv);
  }
  f16* dst = out + ((size_t)b * seq + q0 + r16) * hid + h * kHeadDim + 4 * g;
  *reinterpret_cast<f16x4*>(dst) = w0;
  *reinterpret_cast<f16x4*>(dst + 16) = w1;
}

// ---- unfused pieces with the reference's launcher shapes -------------------

// scores[z, i, j] = scale * sum_d Q[b, i, d] K[b, j, d], z = b*heads + h
// (src/kernels/attention.cu:17-60), fp32 accumulate, fp16 store.
__global__ __launch_bounds__(256) void scores_kernel(const f16* __restrict__ qkv,
                                                     f16* __restrict__ scores, int heads,
                                                     int seq, int ld, int q_off, int k_off_,
                                                     float scale) {
  const int z = blockIdx.y, b = z / heads, h = z % heads;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)seq * seq) return;
  const int i = idx / seq, j = idx % seq;
  const f16* qr = qkv + ((size_t)b * seq + i) * ld + q_off + h * kHeadDim;
  const f16* kr = qkv + ((size_t)b * seq + j) * ld + k_off_ + h * kHeadDim;
  float acc = 0.f;
#pragma unroll
  for (int d = 0; d < kHeadDim; d += 8) {
    const f16x8 a = *reinterpret_cast<const f16x8*>(qr + d);
    const f16x8 c = *reinterpret_cast<const f16x8*>(kr + d);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (float)a[e] * (float)c[e];
  }
  scores[(size_t)z * seq * seq + idx] = (f16)(acc * scale);
}

// Row softmax in place, one wavefront per row (src/kernels/softmax.cu:26-63).
__global__ __launch_bounds__(256) void softmax_kernel(f16* x, int M, int N,
                                                      const int32_t* __restrict__ mask,
                                                      int mask_stride) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  f16* r = x + (size_t)row * N;
  const int32_t* mr = mask ? mask + (mask_stride > 0 ? (size_t)(row / mask_stride) * N : 0)
                           : nullptr;
  float m = -INFINITY;
  for (int i = lane; i < N; i += 64)
    if (!mr || mr[i] != 0) m = fmaxf(m, (float)r[i]);
  m = wave_max(m);
  float s = 0.f;
  for (int i = lane; i < N; i += 64)
    if (!mr || mr[i] != 0) s += __expf((float)r[i] - m);
  s = wave_sum(s);
  const float inv = s > 0.f ? 1.0f / s : 0.f;
  for (int i = lane; i < N; i += 64)
    r[i] = (mr && mr[i] == 0) ? (f16)0.f : (f16)(__expf((float)r[i] - m) * inv);
}

// merged[b*seq+i, h*32+d] = sum_j P[z, i, j] V[b, j, d] (attention.cu:65-93).
__global__ __launch_bounds__(256) void context_kernel(const f16* __restrict__ probs,
                                                      const f16* __restrict__ qkv,
                                                      f16* __restrict__ merged, int heads,
                                                      int seq, int ld, int v_off) {
  const int z = blockIdx.y, b = z / heads, h = z % heads;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= seq * kHeadDim) return;
  const int i = idx / kHeadDim, d = idx % kHeadDim;
  const f16* pr = probs + ((size_t)z * seq + i) * seq;
  const f16* vc = qkv + (size_t)b * seq * ld + v_off + h * kHeadDim + d;
  float acc = 0.f;
  for (int j = 0; j < seq; ++j) acc += (float)pr[j] * (float)vc[(size_t)j * ld];
  merged[((size_t)b * seq + i) * heads * kHeadDim + h * kHeadDim + d] = (f16)acc;
}

}  // namespace

hipError_t attention(const f16* qkv, const int32_t* mask, f16* merged, int batch, int heads,
                     int seq, float scale, hipStream_t s) {
  const float scale_log2 = scale * 1.4426950408889634f;
  if (seq >= 64) {
    dim3 grid((seq + 63) / 64, heads, batch);
    hipLaunchKernelGGL(attention_kernel<4>, grid, dim3(256), 0, s, qkv, mask, merged, seq,
                       heads, scale_log2);
  } else {
    dim3 grid(seq / 16, heads, batch);
    hipLaunchKernelGGL(attention_kernel<1>, grid, dim3(64), 0, s, qkv, mask, merged, seq,
                       heads, scale_log2);
  }
  return hipGetLastError();
}

hipError_t attention_scores(const f16* qkv, f16* scores, int batch, int heads, int seq,
                            int qkv_stride, int q_off, int k_off_, float scale,
                            hipStream_t s) {
  dim3 grid((unsigned)(((size_t)seq * seq + 255) / 256), batch * heads);
  hipLaunchKernelGGL(scores_kernel, grid, dim3(256), 0, s, qkv, scores, heads, seq,
                     qkv_stride, q_off, k_off_, scale);
  return hipGetLastError();
}

hipError_t softmax_rows(f16* x, int M, int N, const int32_t* mask, int mask_stride,
                        hipStream_t s) {
  hipLaunchKernelGGL(softmax_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, M, N, mask,
                     mask_stride);
  return hipGetLastError();
}

hipError_t attention_context(const f16* probs, const f16* qkv, f16* merged, int batch,
                             int heads, int seq, int qkv_stride, int v_off, hipStream_t s) {
  dim3 grid((seq * kHeadDim + 255) / 256, batch * heads);
  hipLaunchKernelGGL(context_kernel, grid, dim3(256), 0, s, probs, qkv, merged, heads, seq,
                     qkv_stride, v_off);
  return hipGetLastError();
}

}  // namespace bbh

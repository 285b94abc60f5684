// Masked multi-head self-attention for head_dim 32, read straight out of the
// fused QKV activations (row stride 3*heads*32, Q | K | V column blocks,
// src/model/weights.h:38-54; strided reads as src/kernels/attention.cu:25-28,
// 74-75) and written straight into the merged (B*S, heads*32) layout
// (attention.cu:87-92).
//
// The reference materialises scores (B*12, S, S) in HBM, runs a separate
// masked softmax over them and a third kernel for P.V
// (src/model/encoder.cu:39-45).  Here one workgroup owns one (sequence, head):
// it stages that head's K (row-major) and V (transposed, [dim][key]) in LDS
// once, then each wavefront walks 32-query tiles with an online softmax, so
// scores never leave the chip (at S = 512 the reference layout is 1.6 GB per
// layer).
//
// Per 32-query x 32-key chunk a wavefront issues four
// v_mfma_f32_32x32x16_f16: two for S^T = K . Q^T (head dims 0-15, 16-31) and
// two for O^T = V^T . P^T (keys 0-15, 16-31).  The 32 K rows of a chunk are
// loaded in the permuted order key_of_row(r) so that the sixteen S^T values a
// lane receives (query lane%32; keys 16*(i/8) + 8*(lane/32) + i%8) are exactly
// the two 8-key groups that lane must supply as operand B of the two P.V
// MFMAs: probabilities go from accumulator to MFMA operand without leaving
// the lane, and V^T is read with one 16-byte LDS load per MFMA.
//
// Softmax in fp32, base 2: the 1/sqrt(32) scale (src/model/encoder.cu:28) and
// log2(e) fold into one FMA before v_exp_f32; the row max needs one
// permlane32 swap (lane ^ 32).  The running max is updated lazily: the
// accumulator is rescaled only when some row's max rises by more than 2^8 in
// probability, so most chunks skip the 16 multiplies and the extra exp.  Row
// sums add the fp16 probabilities (the values the P.V MFMA consumes) with
// v_dot2_f32_f16.  Mask semantics follow src/kernels/softmax.cu:35-62: keys
// with mask 0 are dropped and a query whose keys are all masked gets a zero
// context.  A bitmap of unmasked keys per 32-key chunk, one ballot per 64
// keys, lets fully masked chunks be skipped (their contribution is exactly
// zero) and fully unmasked chunks run without mask arithmetic.
//
// Short sequences are bound by the global round trip: all of a workgroup's
// loads (Q, K, V, mask) are issued before its single barrier, and the output
// goes out through LDS as 16-byte stores of 64 contiguous bytes per row.
// Long sequences are bound by exp + MFMA issue: a wavefront then takes two
// query tiles at once, sharing each K and V^T operand read between them.

#include "kernels.h"

namespace bbh {
namespace {

// Key (within a 32-key chunk) loaded as row r of the S^T tile.
__device__ __forceinline__ int key_of_row(int r) {
  const int a = r >> 3, c = (r >> 2) & 1, b = r & 3;
  return 16 * (a >> 1) + 8 * c + 4 * (a & 1) + b;
}

// Halves offset of 16-byte chunk c (8 head dims) of key row `key` in the K
// tile; the XOR keeps the 16 rows of one operand fetch on distinct banks.
__device__ __forceinline__ int ks_off(int key, int c) {
  return key * 32 + ((c ^ ((key >> 2) & 3)) << 3);
}

// Stride (halves) of a wavefront's 32 x 32 output staging tile in LDS.
constexpr int kStageLd = 40;

size_t attn_lds_bytes(int seq, int staged_waves) {
  const int seqp = (seq + 31) & ~31;
  return (size_t)seqp * 32 * 2 + (size_t)32 * (seqp + 8) * 2 + (size_t)seqp * 4 +
         (size_t)((seqp / 32 + 3) & ~3) * 4 + (size_t)staged_waves * 32 * kStageLd * 2;
}

// Largest step (log2 units) the running row max may lag the true one: while
// every row's chunk max stays within it of the stored max, probabilities are
// taken against the stored max (each at most 2^kLazy, exact in fp16 and fp32)
// and the accumulator is not rescaled.
constexpr float kLazy = 8.f;

// A wavefront works on T query tiles at once (T = 1 or 2): the tiles share
// every K and V^T operand read from LDS, and their two dependency chains
// (scores -> max -> exp -> P.V) interleave.  The workgroup's NW wavefronts
// take tile groups round robin.
// F: 1 stage the output through LDS, 2 put that staging in the K/V area
// (one tile group per wavefront).
// VL: packed sentences (sents[b] gives the rows and length; every token is
// valid, `mask` and `seq` are unused).
template <int NW, int T, int F, bool VL = false>
__global__ __launch_bounds__(64 * NW, T == 2 ? 4 : 6) void attention_kernel(
    const f16* __restrict__ qkv, const int32_t* __restrict__ mask, f16* __restrict__ out,
    int batch, int seq, int heads, float c, const PackedSentence* __restrict__ sents) {
  HIP_DYNAMIC_SHARED(f16, smem);
  // (sequence, head) of this workgroup; all heads of a sequence go to one XCD
  // (workgroup id % 8) back to back, so its QKV rows are fetched into one L2.
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int b = (k / heads) * 8 + x, h = k % heads;
  if (b >= batch) return;
  size_t row0 = (size_t)b * seq;  // first hidden row of the sentence
  if constexpr (VL) {
    const PackedSentence sn = sents[b];
    seq = sn.len;
    row0 = (size_t)sn.row;
    if (seq == 0) return;  // no tokens: nothing to attend, no rows to write
  }
  const int seqp = (seq + 31) & ~31, nch = seqp >> 5, VLD = seqp + 8;
  f16* Ks = smem;                                              // [seqp][32]
  f16* Vt = Ks + seqp * 32;                                    // [32][VLD]
  float* mb = reinterpret_cast<float*>(Vt + 32 * VLD);         // [seqp]: 0 or -inf
  uint32_t* cm = reinterpret_cast<uint32_t*>(mb + seqp);       // [nch]: unmasked-key bitmaps
  f16* stage = reinterpret_cast<f16*>(cm + ((nch + 3) & ~3));  // [NW*T][32][kStageLd]
  const int hid = heads * kHeadDim, ld = 3 * hid;
  const f16* base = qkv + row0 * ld + h * kHeadDim;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r32 = lane & 31, kh = lane >> 5;
  constexpr int NT = 64 * NW;

  // Q of this wavefront's first tile group, issued before the K/V staging so
  // the two global round trips overlap.  Tile t of group g is
  // wave + NW*(T*g + t); a tile past the sequence (T = 2, odd tile count)
  // reads clamped rows and stores nothing.
  f16x8 q0[T], q1[T];
  auto load_q = [&](int g) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int q = (wave + NW * (T * g + t)) * 32 + r32;
      const f16* qrow = base + (size_t)min(q, seq - 1) * ld;
      q0[t] = *reinterpret_cast<const f16x8*>(qrow + 8 * kh);
      q1[t] = *reinterpret_cast<const f16x8*>(qrow + 16 + 8 * kh);
    }
  };
  load_q(0);

  for (int i = tid; i < seqp * 4; i += NT) {  // K: 16 bytes per (key, 8 dims)
    const int key = i >> 2, ch = i & 3;
    f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (key < seq) v = *reinterpret_cast<const f16x8*>(base + (size_t)key * ld + hid + ch * 8);
    *reinterpret_cast<f16x8*>(Ks + ks_off(key, ch)) = v;
  }
  for (int i = tid; i < (seqp / 4) * 8; i += NT) {  // V^T: a 4-key x 4-dim block per thread
    const int dq = i & 7, kq = i >> 3;
    f16x4 r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = 4 * kq + e;
      r[e] = key < seq ? *reinterpret_cast<const f16x4*>(base + (size_t)key * ld + 2 * hid + 4 * dq)
                       : f16x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f16x4 col = {r[0][e], r[1][e], r[2][e], r[3][e]};
      *reinterpret_cast<f16x4*>(Vt + (4 * dq + e) * VLD + 4 * kq) = col;
    }
  }
  if (wave == NW - 1) {  // key bias and bitmaps of unmasked keys, 64 keys per ballot
    const int32_t* mrow = VL ? nullptr : mask + (size_t)b * seq;
    int mv[kMaxPos / 64];
#pragma unroll
    for (int j = 0; j < kMaxPos / 64; ++j) {
      const int key = 64 * j + lane;
      mv[j] = (64 * j < seq && key < seq) ? (VL ? 1 : mrow[key]) : 0;
    }
#pragma unroll
    for (int j = 0; j < kMaxPos / 64; ++j) {
      if (2 * j >= nch) break;
      if (64 * j + lane < seqp) mb[64 * j + lane] = mv[j] != 0 ? 0.f : -INFINITY;
      const unsigned long long on = __ballot(mv[j] != 0);
      if (lane == 0) cm[2 * j] = (uint32_t)on;
      if (lane == 1 && 2 * j + 1 < nch) cm[2 * j + 1] = (uint32_t)(on >> 32);
    }
  }
  __syncthreads();

  const int krow = key_of_row(r32);
  const uint32_t cml = lane < nch ? cm[lane] : 0u;  // lane j holds chunk j's bitmap
  const float lag = kLazy / c;                      // kLazy in raw-score units
  const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const f16x2 ones = {(f16)1.f, (f16)1.f};
  for (int g = 0; wave + NW * T * g < nch; ++g) {
    if (g > 0) load_q(g);
    f32x16 o[T];
    float m[T], l[T];  // running max (raw scores) and sum of the fp16 probabilities
#pragma unroll
    for (int t = 0; t < T; ++t) {
      o[t] = zero;
      m[t] = 0.f;
      l[t] = 0.f;
    }
    bool started = false;
    for (int kc = 0; kc < nch; ++kc) {
      const uint32_t bits = (uint32_t)__builtin_amdgcn_readlane((int)cml, kc);
      if (bits == 0) continue;  // every key of the chunk masked: contributes nothing
      const int key = kc * 32 + krow;
      const f16x8 k0 = *reinterpret_cast<const f16x8*>(Ks + ks_off(key, kh));
      const f16x8 k1 = *reinterpret_cast<const f16x8*>(Ks + ks_off(key, 2 + kh));
      f32x16 s[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        s[t] = mfma32(k0, q0[t], zero);
        s[t] = mfma32(k1, q1[t], s[t]);  // s[i]: key kc*32 + 16*(i/8) + 8*kh + i%8 (raw)
      }
      if (bits != 0xffffffffu) {
        const float* mk = mb + kc * 32 + 8 * kh;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float bias = mk[16 * (i >> 3) + (i & 7)];
#pragma unroll
          for (int t = 0; t < T; ++t) s[t][i] += bias;
        }
      }
      float mx[T];
      bool up = false;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        // IEEE maximum (v_maximum3_f32): scores hold no NaN, and unlike fmaxf
        // it needs no canonicalising v_max_f32 of each MFMA result first.
        float v = __builtin_elementwise_maximum(__builtin_elementwise_maximum(s[t][0], s[t][1]),
                                                s[t][2]);
#pragma unroll
        for (int i = 3; i < 15; i += 2)
          v = __builtin_elementwise_maximum(__builtin_elementwise_maximum(v, s[t][i]), s[t][i + 1]);
        v = __builtin_elementwise_maximum(v, s[t][15]);
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                         false, false);
        mx[t] = __builtin_elementwise_maximum(__uint_as_float(sw[0]),
                                              __uint_as_float(sw[1]));  // finite: a key is unmasked
        up = up || mx[t] > m[t] + lag;
      }
      if (!started) {
#pragma unroll
        for (int t = 0; t < T; ++t) m[t] = mx[t];
        started = true;
      } else if (__ballot(up)) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const float mn = fmaxf(m[t], mx[t]);
          const float corr = __builtin_amdgcn_exp2f((m[t] - mn) * c);
          l[t] *= corr;
          o[t] *= corr;
          m[t] = mn;
        }
      }
      const f16* vrow = Vt + r32 * VLD + kc * 32 + 8 * kh;
      const f16x8 va = *reinterpret_cast<const f16x8*>(vrow);
      const f16x8 vb = *reinterpret_cast<const f16x8*>(vrow + 16);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float mc = m[t] * c;
        f16x8 pa, pb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pa[i] = (f16)__builtin_amdgcn_exp2f(fmaf(s[t][i], c, -mc));
          pb[i] = (f16)__builtin_amdgcn_exp2f(fmaf(s[t][8 + i], c, -mc));
        }
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          l[t] = __builtin_amdgcn_fdot2(f16x2{pa[i], pa[i + 1]}, ones, l[t], false);
          l[t] = __builtin_amdgcn_fdot2(f16x2{pb[i], pb[i + 1]}, ones, l[t], false);
        }
        o[t] = mfma32(va, pa, o[t]);
        o[t] = mfma32(vb, pb, o[t]);
      }
    }
    float inv[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float lt = xor32_sum(l[t]);
      inv[t] = lt > 0.f ? 1.0f / lt : 0.f;
    }
    if constexpr (!(F & 1)) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int q = (wave + NW * (T * g + t)) * 32 + r32;
        if (q < seq) {  // o[i] = O[q][8*(i/4) + 4*kh + i%4]
          f16* dst = out + (row0 + q) * hid + h * kHeadDim + 4 * kh;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            f16x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = (f16)(o[t][4 * j + e] * inv[t]);
            *reinterpret_cast<f16x4*>(dst + 8 * j) = w;
          }
        }
      }
    } else {
      // Through this wavefront's LDS tiles, so that each store instruction
      // writes 16 query rows x 64 contiguous bytes.
      f16* st = stage + wave * T * 32 * kStageLd;
      if ((F & 2) && nch <= NW * T) {  // one group per wavefront: reuse the K/V area once all are done
        if (NW > 1) __syncthreads();
        st = smem + wave * T * 32 * kStageLd;
      }
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f16x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = (f16)(o[t][4 * j + e] * inv[t]);
          *reinterpret_cast<f16x4*>(st + (t * 32 + r32) * kStageLd + 8 * j + 4 * kh) = w;
        }
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int row = 16 * p + (lane >> 2), cc = lane & 3;
          const int q = (wave + NW * (T * g + t)) * 32 + row;
          const f16x8 w = *reinterpret_cast<const f16x8*>(st + (t * 32 + row) * kStageLd + 8 * cc);
          if (q < seq)
            *reinterpret_cast<f16x8*>(out + (row0 + q) * hid + h * kHeadDim + 8 * cc) = w;
        }
    }
  }
  // A packed sentence may have fewer query tiles than the workgroup has
  // wavefronts; those wavefronts still take part in the staging barrier.
  if constexpr (VL && (F & 2)) {
    if (NW > 1 && nch <= NW * T && wave >= nch) __syncthreads();
  }
}

template <int NW, int T, int F, bool VL = false>
hipError_t launch_attention(const f16* qkv, const int32_t* mask, f16* merged, int batch,
                            int heads, int seq, float c, hipStream_t s,
                            const PackedSentence* sents = nullptr) {
  const int tiles = (seq + 31) / 32;  // for VL: of the longest sentence
  const int staged = !(F & 1) || ((F & 2) && tiles <= NW * T) ? 0 : NW * T;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(attention_kernel<NW, T, F, VL>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)attn_lds_bytes(kMaxPos, NW * T));
  if (attr != hipSuccess) return attr;
  const int grid = heads * 8 * ((batch + 7) / 8);
  hipLaunchKernelGGL((attention_kernel<NW, T, F, VL>), dim3(grid), dim3(64 * NW),
                     attn_lds_bytes(seq, staged), s, qkv, mask, merged, batch, seq, heads, c,
                     sents);
  return hipGetLastError();
}

// Workgroup shape by query-tile count (tiles = ceil(seq / 32)).  Up to 7
// tiles: one tile per wavefront, output staged through the K/V area.  8 tiles:
// 4 wavefronts x 2 tiles.  16 tiles: 8 x 2, output staged through the K/V
// area too (16-byte stores of 64-byte row runs; 2% faster at batch 256 x 512
// than the 8-byte stores from the accumulator layout).  9-15: 8 x 1 (a 2-tile
// grouping would leave wavefronts computing empty tiles).  For packed
// sentences the longest one sets the shape.
template <bool VL>
hipError_t attention_any(const f16* qkv, const int32_t* mask, f16* merged, int batch, int heads,
                         int seq, float scale, hipStream_t s, const PackedSentence* sents) {
  const float c = scale * 1.4426950408889634f;  // scores * c are base-2 exponents
  const int tiles = (seq + 31) / 32;
#define BBH_ATT(NW, T, F) \
  launch_attention<NW, T, F, VL>(qkv, mask, merged, batch, heads, seq, c, s, sents)
  if (tiles >= 16) return BBH_ATT(8, 2, 3);
  if (tiles > 8) return BBH_ATT(8, 1, 0);
  if (tiles == 8) return BBH_ATT(4, 2, 3);
  if (tiles >= 4) return BBH_ATT(4, 1, 3);
  if (tiles >= 2) return BBH_ATT(2, 1, 3);
  return BBH_ATT(1, 1, 3);
#undef BBH_ATT
}

}  // namespace

hipError_t attention(const f16* qkv, const int32_t* mask, f16* merged, int batch, int heads,
                     int seq, float scale, hipStream_t s) {
  return attention_any<false>(qkv, mask, merged, batch, heads, seq, scale, s, nullptr);
}

hipError_t attention_packed(const f16* qkv, const PackedSentence* sents, int n, f16* merged,
                            int heads, int max_len, float scale, hipStream_t s) {
  if (n == 0 || max_len == 0) return hipSuccess;
  return attention_any<true>(qkv, nullptr, merged, n, heads, max_len, scale, s, sents);
}

namespace {

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

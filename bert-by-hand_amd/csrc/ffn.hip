// The feed-forward block in one kernel for large M: FFN1 + bias + GELU, then
// FFN2 + bias + residual + LayerNorm, with the (M, 1536) intermediate kept on
// the CU.  The reference's ffn_block (src/model/encoder.cu:53-65) runs two
// launch_matmul calls with the intermediate through memory, then
// launch_layernorm(ffn_out, ..., residual = the block input); at
// batch 256 x seq 512 that intermediate is 403 MB written and read back per
// layer.
//
// Roles.  A workgroup of 12 wavefronts walks blocks of 128 rows.  A 32-row
// strip of the block belongs to three wavefronts on one SIMD:
//  - a producer holds the strip's X (the block input) in VGPRs as the MFMA
//    operand fragments of FFN1's 24 k-steps (96 VGPRs) and makes the
//    intermediate 32 columns at a time (chunk c): one 32x32 accumulator
//    H = X . W1[c]^T, then bias, GELU and fp16 rounding (~250 VALU
//    instructions), then v_permlane32_swap moves H from the accumulator layout
//    (a lane holds 4-column runs of one row) to the operand layout (8
//    consecutive k of one row), and the two fragments go to LDS;
//  - two consumers, one per half of the 384 output columns, hold FFN2's
//    accumulator (32 x 192 fp32, 96 VGPRs each), add H . W2[:, c]^T one chunk
//    behind the producer, and at the end of the block add bias and residual
//    and run the LayerNorm, exchanging row partial sums through LDS.
// The GELU of chunk c runs beside the consumers' MFMAs of chunk c - 1 on the
// same SIMD (MFMA and VALU work of different wavefronts overlap).  Three
// wavefronts per SIMD leave each 168 registers; the kernel uses no AGPRs, so
// all of them are VGPRs (a function with AGPRs gets half its budget in each
// file).
//
// Phases.  Phase k: the producer makes chunk k, the consumers consume chunk
// k - 1; one workgroup barrier ends each phase.  Weights stream in pieces of
// 24 KB: piece 2j = W1 rows 32j' .. 32j'+31 (six 64-wide k slices), piece
// 2j + 1 = W2 k 32j' .. 32j'+31 (all 384 rows), j counting chunks over the
// blocks and j' = j mod 48, in a ring of six filled through global_load_lds by
// the consumers: phase k reads pieces 2k - 1 and 2k and loads pieces 2k + 3
// and 2k + 4, two phases ahead.  H passes through a double buffer.  L2 -> LDS
// traffic is 48 KB per 6.3 MFLOP (128 rows x 32 intermediate columns),
// ~31 B/clk per CU at the MFMA peak.
//
// Arithmetic: FFN1's k order, bias add, GELU polynomial and fp16 rounding are
// those of the GEMM kernels' GELU epilogue; FFN2 accumulates k in their K
// loop's order; bias + residual and the LayerNorm statistics follow the
// N = 384 LayerNorm tiles (mean and squared deviation per group of 96
// columns, the four groups combined in order).  Measured against FFN1 and then FFN2 + residual + LayerNorm of the
// GEMM kernels: equal except on fp16 rounding midpoints (48 of 6.4M outputs at
// 16592 rows, one fp16 step apart, each kernel as often the nearer to a
// float64 evaluation).
//
// Bound: the producer's chain.  Timestamps of one workgroup at M = 131,072
// put a phase at ~3,450 cycles: the producer spends ~1,140 on its 24 MFMAs
// (one dependent chain, sharing the matrix core with the consumers' 24),
// ~1,500 on the GELU and ~300 handing H over, then reaches the barrier; the
// consumers spend 700-1,250 cycles issuing their copies (48 KB a phase at
// ~64 B/clk per CU through the texture path), ~1,100 on their MFMAs, and
// wait.  The matrix core is busy ~45% of the phase.  LDS traffic, ~264 KB a
// phase per CU (every MFMA reads a 1 KB weight fragment; the other operand
// is in registers), stays under what the LDS sustains with two or more
// wavefronts per SIMD (~220-260 B/clk per CU).

#include "kernels.h"
#include "pipe.h"

namespace bbh {
namespace {
namespace ffnf {
constexpr int STRIPS = 4, CONS = 2 * STRIPS;   // producers 0-3; consumers 4-11 (two per strip)
constexpr int NW = STRIPS + CONS, THREADS = 64 * NW;
constexpr int BM = 32 * STRIPS;          // 128 rows per block
constexpr int IC = 32, NC = kFfn / IC;   // intermediate chunk width; 48 chunks per block
constexpr int PIECE = IC * kHidden;      // halves per ring piece (24 KB)
constexpr int RING = 6;
constexpr int CPW = PIECE * 2 / 1024 / CONS;  // 1 KB copies per consumer wavefront per piece
constexpr int KS1 = kHidden / 16;             // FFN1 MFMA k-steps (all of k)
constexpr int KS2 = IC / 16;                  // FFN2 MFMA k-steps per chunk
constexpr int YB = kHidden / 64;              // 32x32 accumulator blocks of a consumer (6)
constexpr int HBUF = STRIPS * KS2 * 64 * 8;   // halves per H buffer: [strip][k-step][lane][8]
constexpr size_t LDS = ((size_t)RING * PIECE + 2 * HBUF) * sizeof(f16);
// From this many rows the kernel runs ahead of FFN1 + FFN2 (MI355X, equal at
// 65536, 8% ahead at 98304 and 131072; 23% behind at 16384, where 128-row
// blocks leave CUs idle).
constexpr int kMinRows = 65536;
static_assert(PIECE * 2 % (1024 * CONS) == 0 && 2 * CPW < 64 && LDS <= kLdsMax, "ring");
static_assert(2 * STRIPS * 4 * 32 * sizeof(float) <= HBUF * sizeof(f16), "LayerNorm partials");
}  // namespace ffnf

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A W2 piece holds 384 rows of 32 k (64 bytes: four 16-byte chunks); logical
// chunk c of row n sits in slot c ^ ((n >> 2) & 3).  Rows n and n + 4 share
// their 16 banks, so the 16 rows of one operand fetch fall on distinct ones.
__device__ __forceinline__ int w2_off(int n, int c) {
  return n * ffnf::IC + ((c ^ ((n >> 2) & 3)) << 3);
}

// Producer, one chunk: h = W1 rows 32c .. 32c+31 . X^T over all 24 k-steps in
// order (P: the W1 piece, six 64-wide slices of 32 rows).
__device__ __forceinline__ void ffn1_chunk(const f16* P, const f16x8 (&x)[ffnf::KS1], f32x16& h) {
  using namespace ffnf;
  const int lane = threadIdx.x & 63, r32 = lane & 31, kh = lane >> 5;
  auto rd = [&](int s) {
    return *reinterpret_cast<const f16x8*>(P + (s >> 2) * 2048 +
                                           Slice<64>::off(r32, 2 * (s & 3) + kh));
  };
  constexpr int PF = 3;  // k-steps read ahead
  f16x8 w[PF + 1];
#pragma unroll
  for (int p = 0; p < PF; ++p) w[p] = rd(p);
#pragma unroll
  for (int s = 0; s < KS1; ++s) {
    if (s + PF < KS1) w[(s + PF) % (PF + 1)] = rd(s + PF);
    h = mfma32(w[s % (PF + 1)], x[s], h);
    if (s + PF < KS1) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
}

// Producer: bias, GELU and fp16 rounding of the chunk's H (bb[j]: the biases
// of the lane's run j), then the operand fragments of FFN2's two k-steps.
// The accumulator holds, in lane (r, kh), the runs hv[j] = H[r][8j + 4kh ..
// +3]; k-step t needs in lane (r, 0) columns 16t .. +7 = hv[2t] of lanes r and
// r + 32, in lane (r, 1) columns 16t + 8 .. +7 = hv[2t+1] of the same two
// lanes: v_permlane32_swap(hv[2t], hv[2t+1]) leaves exactly that in its two
// results.
__device__ __forceinline__ void gelu_operands(const f32x16& h, const f16x4 (&bb)[4],
                                              f16x8 (&hf)[ffnf::KS2]) {
  u32x2 d[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = h[4 * j + e] + (float)bb[j][e];
      v = gelu_poly(v);
      o[e] = to_half(v);
    }
    d[j] = __builtin_bit_cast(u32x2, o);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(d[2 * t][0], d[2 * t + 1][0], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(d[2 * t][1], d[2 * t + 1][1], false, false);
    hf[t] = __builtin_bit_cast(f16x8, u32x4{s0[0], s1[0], s0[1], s1[1]});
  }
}

// Consumer, one chunk: y[b] += W2 rows n0 + 32b .. +31 (k of the chunk) . H^T,
// the chunk's two k-steps in order (P: the W2 piece; n0 the consumer's first
// output column).
__device__ __forceinline__ void ffn2_chunk(const f16* P, int n0, const f16x8 (&hf)[ffnf::KS2],
                                           f32x16 (&y)[ffnf::YB]) {
  using namespace ffnf;
  const int lane = threadIdx.x & 63, r32 = lane & 31, kh = lane >> 5;
  auto rd = [&](int t) {  // MFMA t = s * YB + b
    const int s = t / YB, b = t % YB;
    return *reinterpret_cast<const f16x8*>(P + w2_off(n0 + 32 * b + r32, 2 * s + kh));
  };
  constexpr int T = KS2 * YB, PF = 3;
  f16x8 w[PF + 1];
#pragma unroll
  for (int p = 0; p < PF; ++p) w[p] = rd(p);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t + PF < T) w[(t + PF) % (PF + 1)] = rd(t + PF);
    y[t % YB] = mfma32(w[t % (PF + 1)], hf[t / YB], y[t % YB]);
    if (t + PF < T) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
}

__global__ __launch_bounds__(ffnf::THREADS) void ffn_fused_kernel(
    const f16* X, const f16* __restrict__ W1, const f16* __restrict__ b1,
    const f16* __restrict__ W2, const f16* __restrict__ b2, const f16* __restrict__ gamma,
    const f16* __restrict__ beta, f16* out, int M, float eps) {
  using namespace ffnf;
  HIP_DYNAMIC_SHARED(f16, smem);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r32 = lane & 31, kh = lane >> 5;
  const bool producer = wave < STRIPS;
  const int strip = wave % STRIPS;  // wavefront w runs on SIMD w % 4: a strip's three share one
  const int cons = wave - STRIPS;   // consumer index 0 .. 7
  const int half = cons / STRIPS;   // consumer: output columns 192 half .. +191
  f16* ring = smem;
  f16* hbuf = smem + RING * PIECE;

  const int nblk = (M + BM - 1) / BM;
  const int my = (int)blockIdx.x < nblk ? (nblk - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int nchunks = my * NC, npieces = 2 * nchunks;
  auto row0 = [&](int j) {  // first row of this wavefront's strip in the block of chunk j
    return ((int)blockIdx.x + (j / NC) * (int)gridDim.x) * BM + 32 * strip;
  };

  // Consumer copies (q = CONS i + cons, i = 0 .. CPW - 1).  W1 piece: copy q
  // fills rows 8 (q % 4) .. +7 of slice q / 4 (32 rows x 64 k); lane l lands
  // at row 8 (q % 4) + l / 8, slot l % 8, fetching logical chunk
  // (l % 8) ^ f(row), f(row) = (4 (q & 1) + l / 16) & 7.  W2 piece: copy q
  // fills rows 16 q .. +15; lane l lands at row 16 q + l / 4, slot l % 4,
  // fetching logical chunk (l % 4) ^ (l / 16).  q & 1 = cons & 1 for every
  // copy of a wavefront, so each needs one per-lane offset.
  const __amdgpu_buffer_rsrc_t rW1 = buffer_of(W1, (uint32_t)kFfn * kHidden * 2u);
  const __amdgpu_buffer_rsrc_t rW2 = buffer_of(W2, (uint32_t)kHidden * kFfn * 2u);
  const int cl1 = (lane & 7) ^ ((4 * (cons & 1) + (lane >> 4)) & 7);
  const uint32_t lo1 = ((lane >> 3) * kHidden + cl1 * 8) * 2u;
  const uint32_t lo2 = ((lane >> 2) * kFfn + (((lane & 3) ^ (lane >> 4)) << 3)) * 2u;
  auto issue = [&](int g) {  // piece g into ring slot g % RING
    const int c = (g >> 1) % NC;
    f16* buf = ring + (g % RING) * PIECE;
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
      const int q = i * CONS + cons;
      if ((g & 1) == 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rW1, (__attribute__((address_space(3))) void*)(buf + q * 512), 16, (int)lo1,
            ((32 * c + 8 * (q & 3)) * kHidden + 64 * (q >> 2)) * 2, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rW2, (__attribute__((address_space(3))) void*)(buf + q * 512), 16, (int)lo2,
            (16 * q * kFfn + IC * c) * 2, 0, 0);
    }
  };
  // Phase k ends a block (the consumers' epilogue, with two extra barriers
  // for the LayerNorm partials) when chunk k - 1 is a block's last.
  auto epilogue_phase = [&](int k) { return k >= 1 && (k - 1) % NC == NC - 1; };

  // Prologue: pieces 0 (phase 0), 1 and 2 (phase 1); phase 0 waits for piece 0.
  if (!producer) {
#pragma unroll
    for (int g = 0; g < 3; ++g)
      if (g < npieces) issue(g);
    if (npieces > 2)
      wait_vm<2 * CPW>();
    else
      wait_vm<0>();
  }
  lds_barrier();

  if (producer) {
    f16x8 x[KS1];
#pragma unroll 1
    for (int k = 0; k <= nchunks; ++k) {
      if (k < nchunks) {
        const int c = k % NC;
        f16x4 bb[4];  // b1 of the chunk, this lane's runs
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bb[j] = *reinterpret_cast<const f16x4*>(b1 + IC * c + 8 * j + 4 * kh);
        if (c == 0) {
          // The strip's X fragments: lane (r, kh) holds X[r][16 s + 8 kh .. +7]
          // for k-step s; rows past M read row M - 1.
          const f16* xr = X + (size_t)min(row0(k) + r32, M - 1) * kHidden + 8 * kh;
#pragma unroll
          for (int s = 0; s < KS1; ++s) x[s] = *reinterpret_cast<const f16x8*>(xr + 16 * s);
        }
        f32x16 h;
#pragma unroll
        for (int i = 0; i < 16; ++i) h[i] = 0.f;
        ffn1_chunk(ring + ((2 * k) % RING) * PIECE, x, h);
        f16x8 hf[KS2];
        gelu_operands(h, bb, hf);
        f16* hb = hbuf + (k & 1) * HBUF + strip * (KS2 * 512) + lane * 8;
#pragma unroll
        for (int t = 0; t < KS2; ++t) *reinterpret_cast<f16x8*>(hb + t * 512) = hf[t];
      }
      if (epilogue_phase(k)) {  // the consumers' two LayerNorm barriers
        lds_barrier();
        lds_barrier();
      }
      lds_barrier();
    }
  } else {
    f32x16 y[YB];
    const int n0 = 192 * half;
#pragma unroll 1
    for (int k = 0; k <= nchunks; ++k) {
      // Pieces 2k + 3 and 2k + 4 into the slots of pieces 2k - 3 and 2k - 2,
      // which phase k - 1 consumed.
      const int g = 2 * k + 3;
      if (g < npieces) issue(g);
      if (g + 1 < npieces) issue(g + 1);
      if (k >= 1) {
        const int j = k - 1, c = j % NC;
        if (c == 0) {
#pragma unroll
          for (int b = 0; b < YB; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) y[b][i] = 0.f;
        }
        f16x8 hf[KS2];
        const f16* hb = hbuf + (j & 1) * HBUF + strip * (KS2 * 512) + lane * 8;
#pragma unroll
        for (int t = 0; t < KS2; ++t) hf[t] = *reinterpret_cast<const f16x8*>(hb + t * 512);
        ffn2_chunk(ring + ((2 * j + 1) % RING) * PIECE, n0, hf, y);
      }
      if (epilogue_phase(k)) {
        // y += b2 + residual (X, the block input), then the LayerNorm.  Lane
        // (r, kh) holds columns n0 + 32 b + 8 jj + 4 kh .. +3 of row r in
        // y[b][4 jj ..].
        const int row = row0(k - 1) + r32;
        const f16* xr = X + (size_t)min(row, M - 1) * kHidden + n0 + 4 * kh;
#pragma unroll
        for (int b = 0; b < YB; ++b)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int n = 32 * b + 8 * jj;
            const f16x4 rv = *reinterpret_cast<const f16x4*>(xr + n);
            const f16x4 bv = *reinterpret_cast<const f16x4*>(b2 + n0 + n + 4 * kh);
#pragma unroll
            for (int e = 0; e < 4; ++e) y[b][4 * jj + e] += (float)bv[e] + (float)rv[e];
            // One block's loads in flight at a time: registers are short here.
            if (jj == 3) __builtin_amdgcn_sched_barrier(0);
          }
        // Row statistics as the N = 384 LayerNorm tiles take them: per
        // 96-column group g (this consumer holds groups 2 half, 2 half + 1)
        // the mean and squared deviation over a lane's 48 values plus lane ^
        // 32's, then the four groups combined in order as equal-size groups
        // (Chan et al.).  The pairs pass through the H buffer that phase
        // k - 1 filled (free once every consumer has read it: first barrier).
        float2* red = reinterpret_cast<float2*>(hbuf + ((k - 1) & 1) * HBUF) + strip * 128;
        float mw[2], qw[2];
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
          float sg = 0.f;
#pragma unroll
          for (int b = 3 * gg; b < 3 * gg + 3; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) sg += y[b][i];
          mw[gg] = xor32_sum(sg) * (1.0f / 96);
          float qg = 0.f;
#pragma unroll
          for (int b = 3 * gg; b < 3 * gg + 3; ++b)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const float d = y[b][i] - mw[gg];
              qg += d * d;
            }
          qw[gg] = xor32_sum(qg);
        }
        lds_barrier();
        if (kh == 0) {
          red[(2 * half) * 32 + r32] = make_float2(mw[0], qw[0]);
          red[(2 * half + 1) * 32 + r32] = make_float2(mw[1], qw[1]);
        }
        lds_barrier();
        float tsum = 0.f;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) tsum += red[g4 * 32 + r32].x;
        const float mean = tsum * (1.0f / 4);
        float tq = 0.f, dd = 0.f;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const float2 pw = red[g4 * 32 + r32];
          const float d = pw.x - mean;
          tq += pw.y;
          dd += d * d;
        }
        const float rstd = rsqrtf(fmaf(96.f, dd, tq) * (1.0f / kHidden) + eps);
#pragma unroll
        for (int b = 0; b < YB; ++b)
#pragma unroll
          for (int i = 0; i < 16; ++i) y[b][i] -= mean;  // as the tiles: (v - mean) * rstd * g + b
#pragma unroll
        for (int b = 0; b < YB; ++b)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int n = n0 + 32 * b + 8 * jj + 4 * kh;
            const f16x4 gv = *reinterpret_cast<const f16x4*>(gamma + n);
            const f16x4 be = *reinterpret_cast<const f16x4*>(beta + n);
            f16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              o[e] = to_half(y[b][4 * jj + e] * rstd * (float)gv[e] + (float)be[e]);
            if (row < M) *reinterpret_cast<f16x4*>(out + (size_t)row * kHidden + n) = o;
            if (jj == 3) __builtin_amdgcn_sched_barrier(0);
          }
      }
      // Pieces 2k + 1 and 2k + 2 (phase k + 1) landed: only this phase's
      // copies may still be in flight (copies retire in issue order; later
      // loads and stores only make the wait stricter).
      if (g + 1 < npieces)
        wait_vm<2 * CPW>();
      else if (g < npieces)
        wait_vm<CPW>();
      else
        wait_vm<0>();
      lds_barrier();
    }
  }
}

}  // namespace

bool ffn_fused_ok(int M) { return M >= ffnf::kMinRows; }

hipError_t ffn_fused(const f16* X, const f16* W1, const f16* b1, const f16* W2, const f16* b2,
                     const f16* gamma, const f16* beta, f16* out, int M, float eps, hipStream_t s) {
  using namespace ffnf;
  if (M <= 0) return hipSuccess;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(ffn_fused_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS);
  if (attr != hipSuccess) return attr;
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  // One workgroup per CU (ring and H buffers fill its LDS), each walking
  // blocks blockIdx.x, blockIdx.x + grid, ...
  const int nblk = (M + BM - 1) / BM;
  hipLaunchKernelGGL(ffn_fused_kernel, dim3(std::min(nblk, cus)), dim3(THREADS), LDS, s, X, W1,
                     b1, W2, b2, gamma, beta, out, M, eps);
  return hipGetLastError();
}

}  // namespace bbh

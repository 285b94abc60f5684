// Linear layers of the encoder on the CDNA4 matrix cores.
//
// Every Linear in the path is C(M,N) = A(M,K) . W(N,K)^T with the torch
// (out, in) weight layout (reference: src/kernels/matmul.h:1-13), so both
// operands are K-contiguous.  fp16 operands, fp32 accumulation (the reference
// accumulates in fp16 on GeForce, src/kernels/matmul.cu:97-110; CDNA4 runs
// fp32 accumulate at full rate).
//
// Matrix-core instruction: v_mfma_f32_32x32x16_f16.  Measured on MI355X it
// sustains ~2.15 PFLOP/s against ~1.44 for the 16x16x32 form, so every tile
// here is built from 32x32 blocks.  The kernels compute the transposed tile
// D(n, m) = W . A^T: lane l then holds, per 32x32 block, four runs of four
// consecutive output columns n of one row m.
//
// Operand pipeline: a workgroup of 4 wavefronts owns a BM x BN output tile
// and walks K in 64-wide slices.  Slices are copied global -> LDS with
// global_load_lds_dwordx4 (16 bytes per lane, no register staging) into two
// rings: the activations A, streamed from HBM, run SA-1 slices ahead (their
// HBM latency is what a single shared ring exposes), the weights W, resident
// in L2, SW-1 slices ahead (SW = 2 in every configuration in the table: deeper
// W rings measured no faster); one barrier per slice.  The other pipeline
// stages PD slices per thread in VGPRs and double-buffers one LDS tile.  Within a slice, row r is
// 128 bytes = 8 chunks of 16 bytes and logical chunk c sits in slot
// c ^ ((r >> 1) & 7): the 16 rows one MFMA operand fetch touches per LDS cycle
// then hit 16 distinct bank groups.
//
// Tile order is XCD-aware: workgroup b runs on XCD b % 8, and the N-tiles of
// one M-tile are given to consecutive workgroups of the same XCD so the A
// rows are fetched from HBM once per XCD and re-read from that XCD's L2.
//
// Epilogues (fp32, then staged through LDS as fp16 for 16-byte coalesced
// stores): bias; bias + exact-erf GELU (src/kernels/matmul.cu:23-30);
// bias + residual; bias + residual + LayerNorm over the full 384-wide row
// (folds the reference's separate launch_layernorm(x, ..., residual),
// src/model/encoder.cu:47-50,61-64, src/kernels/layernorm.cu:17-59).

#include <type_traits>

#include "kernels.h"
#include "pipe.h"

namespace bbh {
namespace {

// kFold / kFoldGelu and kResStats: the two sides of LnCarry (kernels.h).
enum Epi { kBias = 0, kGelu = 1, kResidual = 2, kLayerNorm = 3, kFold = 4, kFoldGelu = 5, kResStats = 6 };

template <int BM_, int BN_, int WM_, int WN_, int SA_, int PD_ = 0, int SW_ = 2>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, SA = SA_, SW = SW_, BK = 64;
  // PD_ > 0: register prefetch depth (mainloop_reg); PD_ < 0: the copy-ring
  // loop with KPB = -PD_ K slices per barrier (mainloop_multi).
  static constexpr int PD = PD_ > 0 ? PD_ : 0;
  static constexpr int KPB = PD_ < 0 ? -PD_ : 1;
  using L = Slice<64>;
  static constexpr int NW = WM * WN, THREADS = 64 * NW;  // 4 or 8 wavefronts
  static constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
  static constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 blocks per wave
  static constexpr int LA = BM / (8 * NW), LW = BN / (8 * NW);  // copies per thread per slice
  static constexpr int A_STAGE = BM * BK, W_STAGE = BN * BK;  // halves per slice
  static constexpr int W_BASE = SA * A_STAGE;                 // W ring follows the A ring
  static constexpr int OUT_LD = BN + 8;                       // padded row of the fp16 output tile
  static constexpr int CA = BM * 8 / THREADS, CW = BN * 8 / THREADS;  // 16-B chunks per thread
  static constexpr size_t RING = PD > 0 ? (size_t)2 * (A_STAGE + W_STAGE) * sizeof(f16)
                                        : (size_t)(SA * A_STAGE + SW * W_STAGE) * sizeof(f16);
  static constexpr size_t RED = 2 * WN * BM * sizeof(float);  // LayerNorm row partials
  // The fp16 output tile is staged through LDS in NPASS row passes (one per
  // wave row when the whole tile does not fit next to the partials).
  static constexpr int NPASS = ((size_t)BM * OUT_LD * sizeof(f16) + RED <= kLdsMax) ? 1 : WM;
  static constexpr size_t OUT = (size_t)(BM / NPASS) * OUT_LD * sizeof(f16) + RED;
  static constexpr size_t LDS = RING > OUT ? RING : OUT;
  static_assert(NW == 4 || NW == 6 || NW == 8, "four, six or eight wavefronts");
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile is whole 32x32 blocks");
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "load distribution");
  static_assert(SA >= 2 && SW >= 2, "ring depths");
  static_assert(KPB == 1 || (PD == 0 && SA == 2 * KPB && SW == 2 * KPB),
                "KPB slices per barrier: rings of 2 * KPB slices");
  // vmcnt that may stay outstanding when slice kt must have landed: the
  // copies issued after the later of W(kt) and A(kt) (W is issued first in
  // each iteration).
  static constexpr int VM_AHEAD = ((SA < SW ? SA : SW) - 2) * (LA + LW) + (SW < SA ? LA : 0);
  static_assert(VM_AHEAD < 64, "vmcnt range");
  static_assert(LDS <= kLdsMax, "LDS");
  static_assert(PD == 0 || (BM * 8 % THREADS == 0 && BN * 8 % THREADS == 0), "chunks");
};

// Copying one 64-wide K slice of ROWS K-contiguous rows into LDS: each
// wavefront instruction fills 1 KB = 8 rows; lane i lands at row i / 8, slot
// i % 8 of them, so it fetches the logical chunk that belongs in that slot.
// Rows at or past `valid` are read clamped to row valid-1.  row_offsets gives
// off[j] = byte offset of this lane's chunk of copy j from the slice base,
// computed once per tile; issue_rows_at then copies a slice through a buffer
// resource, the slice's K offset being the instruction's scalar operand.  A
// K loop so pays no per-lane address arithmetic per copy (on the SIMD issue
// the MFMAs share: ~65 VALU instructions per wavefront per slice before).
template <int ROWS, int NW>
__device__ __forceinline__ void row_offsets(int ld, int valid, uint32_t (&off)[ROWS / (8 * NW)]) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < ROWS / (8 * NW); ++j) {
    const int r = (wave * (ROWS / (8 * NW)) + j) * 8 + (lane >> 3);
    off[j] = (uint32_t)(min(r, valid - 1) * ld + (((lane & 7) ^ Slice<64>::f(r)) << 3)) * 2u;
  }
}

// One slice's copies: lane chunk offsets from row_offsets, slice offset
// `soff` bytes (wave-uniform).
template <int ROWS, int NW>
__device__ __forceinline__ void issue_rows_at(__amdgpu_buffer_rsrc_t src, uint32_t soff,
                                              const uint32_t (&off)[ROWS / (8 * NW)], f16* buf) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
  for (int j = 0; j < ROWS / (8 * NW); ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        src, (__attribute__((address_space(3))) void*)(buf + (wave * (ROWS / (8 * NW)) + j) * 8 * 64),
        16, (int)off[j], (int)soff, 0, 0);
}

// Scheduling groups: (one DS read, then ~Q/R MFMAs) x R.
template <int R, int Q, int I = 0>
__device__ __forceinline__ void interleave() {
  if constexpr (I < R) {
    constexpr int n = (I < Q % R) ? Q / R + 1 : Q / R;
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x008, n, 0);
    interleave<R, Q, I + 1>();
  }
}

// MFMA work of one 64-wide K slice staged in LDS (sA: BM rows, sW: BN rows).
// The fragments of k-step s+PF are read from LDS while the MFMAs of step s
// run (a ring of PF+1 fragment sets), so a step waits only for reads issued
// PF steps earlier; the reads are spread over the MFMAs of a step.
#ifndef BBH_LDS_PF
#define BBH_LDS_PF 1  // 2 measured no faster and costs registers
#endif
template <class C>
__device__ __forceinline__ void compute_slice(const f16* sA, const f16* sW,
                                              f32x16 (&acc)[C::FM][C::FN]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int r32 = lane & 31, kh = lane >> 5;
  constexpr int KS = C::BK / 16;    // MFMA k-steps per slice
  constexpr int R = C::FM + C::FN;  // LDS fragment reads per k-step
  constexpr int Q = C::FM * C::FN;  // MFMAs per k-step
  constexpr int PF = BBH_LDS_PF < KS ? BBH_LDS_PF : KS - 1;
  constexpr int NB = PF + 1;
  f16x8 a[NB][C::FM], w[NB][C::FN];
  auto rd = [&](int s, f16x8(&aa)[C::FM], f16x8(&ww)[C::FN]) {
#pragma unroll
    for (int fm = 0; fm < C::FM; ++fm)
      aa[fm] = *reinterpret_cast<const f16x8*>(sA + C::L::off(wm * C::TM + fm * 32 + r32, 2 * s + kh));
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn)
      ww[fn] = *reinterpret_cast<const f16x8*>(sW + C::L::off(wn * C::TN + fn * 32 + r32, 2 * s + kh));
  };
#pragma unroll
  for (int p = 0; p < PF; ++p) rd(p, a[p], w[p]);
  __builtin_amdgcn_sched_group_barrier(0x100, R * PF, 0);  // the first PF steps' reads first
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (s + PF < KS) rd(s + PF, a[(s + PF) % NB], w[(s + PF) % NB]);
#pragma unroll
    for (int fm = 0; fm < C::FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < C::FN; ++fn)
        acc[fm][fn] = mfma32(w[s % NB][fn], a[s % NB][fm], acc[fm][fn]);
    if (s + PF < KS)
      interleave<R, Q>();  // spread step s+PF's R fragment reads over these Q MFMAs
    else
      __builtin_amdgcn_sched_group_barrier(0x008, Q, 0);
  }
}

// The K loop.  A (activations, streamed from HBM) and W (weights, L2
// resident) have separate LDS rings: A runs SA-1 slices ahead, W one slice
// ahead.  Iteration j issues W(j+1) and then A(j+SA-1); because the DMA
// counter retires in issue order, waiting for W(kt) only has to allow the
// LA copies of A(kt+SA-2) issued right after it to stay in flight, and A(kt)
// (issued at j <= kt-2) is then complete too.
// On return acc[fm][fn][i] = D(n, m) with
//   n = n0 + wn*TN + fn*32 + 8*(i/4) + 4*(lane/32) + i%4,
//   m = m0 + wm*TM + fm*32 + lane%32.
template <class C>
__device__ __forceinline__ void mainloop(const f16* __restrict__ A, const f16* __restrict__ W,
                                         int M, int K, int m0, int n0, f16* smem,
                                         f32x16 (&acc)[C::FM][C::FN]) {
#pragma unroll
  for (int fm = 0; fm < C::FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[fm][fn][i] = 0.f;

  const int KT = K / C::BK;
  f16* ringA = smem;
  f16* ringW = smem + C::W_BASE;
  const f16* a0 = A + (size_t)m0 * K;
  const f16* w0 = W + (size_t)n0 * K;
  // The launcher keeps M * K * 2 below 2^31 (row chunks), so every byte offset fits.
  uint32_t offA[C::LA], offW[C::LW];
  row_offsets<C::BM, C::NW>(K, M - m0, offA);
  row_offsets<C::BN, C::NW>(K, C::BN, offW);
  const __amdgpu_buffer_rsrc_t rA = buffer_of(a0, (uint32_t)(M - m0) * K * 2u);
  const __amdgpu_buffer_rsrc_t rW = buffer_of(w0, (uint32_t)C::BN * K * 2u);
  auto issueA = [&](int s) {
    issue_rows_at<C::BM, C::NW>(rA, s * C::BK * 2, offA, ringA + (s % C::SA) * C::A_STAGE);
  };
  auto issueW = [&](int s) {
    issue_rows_at<C::BN, C::NW>(rW, s * C::BK * 2, offW, ringW + (s % C::SW) * C::W_STAGE);
  };
  // Slice s of W is issued SW-1 iterations and slice s of A SA-1 iterations
  // before it is consumed; the prologue is iterations j = 1-max(SA,SW) .. -1
  // of the same schedule.
  constexpr int S = C::SA > C::SW ? C::SA : C::SW;
#pragma unroll
  for (int j = 1 - S; j <= -1; ++j) {
    if (j + C::SW - 1 >= 0 && j + C::SW - 1 < KT) issueW(j + C::SW - 1);
    if (j + C::SA - 1 >= 0 && j + C::SA - 1 < KT) issueA(j + C::SA - 1);
  }

  for (int kt = 0; kt < KT; ++kt) {
    if (C::VM_AHEAD > 0 && kt + S - 2 < KT)
      wait_vm<C::VM_AHEAD>();
    else
      wait_vm<0>();
    lds_barrier();  // slice kt visible to all; slice kt-1 fully consumed
    if (kt + C::SW - 1 < KT) issueW(kt + C::SW - 1);
    if (kt + C::SA - 1 < KT) issueA(kt + C::SA - 1);
    const f16* sA = ringA + (kt % C::SA) * C::A_STAGE;
    const f16* sW = ringW + (kt % C::SW) * C::W_STAGE;
    compute_slice<C>(sA, sW, acc);
  }
  lds_barrier();  // ring free for the epilogue
}

// The copy-ring K loop with KPB slices per barrier: rings of 2 * KPB slices
// for A and W.  Iteration k0 waits for slices k0 .. k0+KPB-1 (the copies
// issued one iteration earlier), passes one barrier, refills the KPB slots
// that iteration k0-KPB read with slices k0+KPB .., and runs its KPB slices,
// so the copy wait, the barrier and the copy issue are paid once per KPB
// slices instead of once per slice.  Same k order and accumulation as
// mainloop.
template <class C>
__device__ __forceinline__ void mainloop_multi(const f16* __restrict__ A,
                                               const f16* __restrict__ W, int M, int K, int m0,
                                               int n0, f16* smem, f32x16 (&acc)[C::FM][C::FN]) {
#pragma unroll
  for (int fm = 0; fm < C::FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[fm][fn][i] = 0.f;

  constexpr int P = C::KPB;
  const int KT = K / C::BK;
  f16* ringA = smem;
  f16* ringW = smem + C::W_BASE;
  const f16* a0 = A + (size_t)m0 * K;
  const f16* w0 = W + (size_t)n0 * K;
  uint32_t offA[C::LA], offW[C::LW];
  row_offsets<C::BM, C::NW>(K, M - m0, offA);
  row_offsets<C::BN, C::NW>(K, C::BN, offW);
  const __amdgpu_buffer_rsrc_t rA = buffer_of(a0, (uint32_t)(M - m0) * K * 2u);
  const __amdgpu_buffer_rsrc_t rW = buffer_of(w0, (uint32_t)C::BN * K * 2u);
  auto issue = [&](int s) {
    issue_rows_at<C::BN, C::NW>(rW, s * C::BK * 2, offW, ringW + (s % C::SW) * C::W_STAGE);
    issue_rows_at<C::BM, C::NW>(rA, s * C::BK * 2, offA, ringA + (s % C::SA) * C::A_STAGE);
  };
#pragma unroll
  for (int d = 0; d < P; ++d)
    if (d < KT) issue(d);
  for (int k0 = 0; k0 < KT; k0 += P) {
    wait_vm<0>();
    lds_barrier();  // slices k0 .. k0+P-1 visible to all; k0-P .. k0-1 consumed
#pragma unroll
    for (int d = 0; d < P; ++d)
      if (k0 + P + d < KT) issue(k0 + P + d);
#pragma unroll
    for (int d = 0; d < P; ++d)
      if (k0 + d < KT)
        compute_slice<C>(ringA + ((k0 + d) % C::SA) * C::A_STAGE,
                         ringW + ((k0 + d) % C::SW) * C::W_STAGE, acc);
  }
  lds_barrier();  // ring free for the epilogue
}

// The K loop with register staging: each thread keeps the 16-byte chunks of
// the next PD slices in flight in VGPRs (the register file holds far more
// in-flight bytes than LDS), then writes one slice per iteration into a
// double-buffered LDS tile.  The compiler's own counters order the register
// loads; buffer kt&1 was last read in iteration kt-2, before barrier kt-1.
template <class C>
__device__ __forceinline__ void mainloop_reg(const f16* __restrict__ A,
                                             const f16* __restrict__ W, int M, int K, int m0,
                                             int n0, f16* smem, f32x16 (&acc)[C::FM][C::FN]) {
#pragma unroll
  for (int fm = 0; fm < C::FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[fm][fn][i] = 0.f;
  constexpr int D = C::PD, CA = C::CA, CW = C::CW;
  const int KT = K / C::BK, tid = threadIdx.x, last = M - m0 - 1;
  const f16* a0 = A + (size_t)m0 * K;
  const f16* w0 = W + (size_t)n0 * K;
  f16x8 ra[D][CA], rw[D][CW];
  // Lane byte offsets of each chunk from the slice base, computed once; a
  // slice adds its offset as the buffer instruction's scalar operand.  The
  // launcher keeps M * K * 2 below 2^31.
  uint32_t offA[CA], offW[CW];
#pragma unroll
  for (int i = 0; i < CA; ++i) {
    const int c = tid + i * C::THREADS;
    offA[i] = ((uint32_t)min(c >> 3, last) * K + (c & 7) * 8) * 2u;
  }
#pragma unroll
  for (int i = 0; i < CW; ++i) {
    const int c = tid + i * C::THREADS;
    offW[i] = ((uint32_t)(c >> 3) * K + (c & 7) * 8) * 2u;
  }
  const __amdgpu_buffer_rsrc_t rA = buffer_of(a0, (uint32_t)(M - m0) * K * 2u);
  const __amdgpu_buffer_rsrc_t rW = buffer_of(w0, (uint32_t)C::BN * K * 2u);
  auto load = [&](int s, f16x8(&xa)[CA], f16x8(&xw)[CW]) {
#pragma unroll
    for (int i = 0; i < CA; ++i)
      xa[i] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(rA, (int)offA[i], s * C::BK * 2, 0));
#pragma unroll
    for (int i = 0; i < CW; ++i)
      xw[i] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(rW, (int)offW[i], s * C::BK * 2, 0));
  };
  auto store = [&](int buf, const f16x8(&xa)[CA], const f16x8(&xw)[CW]) {
    f16* sA = smem + buf * (C::A_STAGE + C::W_STAGE);
    f16* sW = sA + C::A_STAGE;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int c = tid + i * C::THREADS;
      *reinterpret_cast<f16x8*>(sA + C::L::off(c >> 3, c & 7)) = xa[i];
    }
#pragma unroll
    for (int i = 0; i < CW; ++i) {
      const int c = tid + i * C::THREADS;
      *reinterpret_cast<f16x8*>(sW + C::L::off(c >> 3, c & 7)) = xw[i];
    }
  };
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < KT) load(d, ra[d], rw[d]);
  for (int kt0 = 0; kt0 < KT; kt0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int kt = kt0 + d;
      if (kt < KT) {
        store(kt & 1, ra[d], rw[d]);
        if (kt + D < KT) load(kt + D, ra[d], rw[d]);
        lds_barrier();
        const f16* sA = smem + (kt & 1) * (C::A_STAGE + C::W_STAGE);
        compute_slice<C>(sA, sA + C::A_STAGE, acc);
      }
    }
  }
  lds_barrier();  // LDS free for the epilogue
}

// Tile coordinates from the workgroup id, XCD-aware (see header).
__device__ __forceinline__ bool tile_of(int nb, int mb, int& mi, int& ni) {
  const int b = blockIdx.x, x = b & 7, k = b >> 3;
  ni = k % nb;
  mi = (k / nb) * 8 + x;
  return mi < mb;
}

// Write ROWS rows of the output tile, staged in LDS as ROWS x OUT_LD fp16,
// to C rows m0.. with 16-byte stores.
// A thread's residual chunks of the tile (store_rows' mapping), loaded
// before the K loop so that their latency hides behind it instead of
// following it: tiles staged in one pass with at most four chunks a thread.
template <class C>
struct ResidualAhead {
  static constexpr int CPR = C::BN / 8;
  static constexpr int PER = (C::BM * CPR + C::THREADS - 1) / C::THREADS;
  static constexpr bool kOn = C::NPASS == 1 && PER <= 4;
  f16x8 r[kOn ? PER : 1];
  __device__ __forceinline__ void load(const f16* residual, int ldc, int M, int m0, int n0) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int idx = threadIdx.x + q * C::THREADS;
      const int row = idx / CPR, c = idx % CPR;
      if (idx < C::BM * CPR && m0 + row < M) {
        r[q] = *reinterpret_cast<const f16x8*>(residual + (size_t)(m0 + row) * ldc + n0 + c * 8);
      }
    }
  }
};

template <class C, int ROWS>
__device__ __forceinline__ void store_rows(const f16* tile, f16* __restrict__ out, int ldc, int M,
                                           int m0, int n0, const f16* residual,
                                           const f16x8* ahead = nullptr) {
  constexpr int CPR = C::BN / 8;
  constexpr int PER = (ROWS * CPR + C::THREADS - 1) / C::THREADS;
  // Unrolled so the residual loads of several rows are in flight together
  // (by 4 when the tile is staged in passes and other accumulators are live).
  constexpr int kUnroll = C::NPASS == 1 ? PER : 4;
#pragma unroll kUnroll
  for (int q = 0; q < PER; ++q) {
    const int idx = threadIdx.x + q * C::THREADS;
    const int r = idx / CPR, c = idx % CPR;
    if (idx < ROWS * CPR && m0 + r < M) {
      f16x8 v = *reinterpret_cast<const f16x8*>(tile + r * C::OUT_LD + c * 8);
      if (residual) {
        const f16x8 rv =
            ahead ? ahead[q]
                  : *reinterpret_cast<const f16x8*>(residual + (size_t)(m0 + r) * ldc + n0 + c * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (f16)((float)v[i] + (float)rv[i]);
      }
      *reinterpret_cast<f16x8*>(out + (size_t)(m0 + r) * ldc + n0 + c * 8) = v;
    }
  }
}

// store_rows for kResStats: the residual, brought through its LayerNorm when
// cy.mr_in is given (the rows' (mean, rstd) and the columns' gamma / beta
// staged in LDS: rmr for the pass's rows, rgb), is added in fp32 to the fp16
// tile value; then the mean
// and the sum of squared deviations of each stored fp16 row over each
// 64-column group go to cy.st_out (pair n / 64 of the row), summed in the
// same order whatever the tile width, so the statistics, and all that is
// computed from them, do not depend on the tile.  A row's CPR = BN / 8
// threads are consecutive lanes of one wavefront, so every lane of such a
// group takes the same branches.
template <class C, int ROWS>
__device__ __forceinline__ void store_rows_stats(const f16* tile, f16* __restrict__ out, int M,
                                                 int m0, int n0, const f16* residual,
                                                 const float2* rmr, const f16* rgb,
                                                 const LnCarry& cy,
                                                 const ResidualAhead<C>* ahead) {
  constexpr int CPR = C::BN / 8, N = kHidden;
  static_assert(CPR == 8 || CPR == 16, "a row's chunks on 8 or 16 lanes");
  constexpr int PER = (ROWS * CPR + C::THREADS - 1) / C::THREADS;
  constexpr int kUnroll = C::NPASS == 1 ? PER : 4;
  static_assert(C::THREADS % CPR == 0, "a thread keeps its chunk column");
  // A thread's chunks all sit in chunk column threadIdx.x % CPR: gamma and
  // beta of its 8 columns once.
  const int c = threadIdx.x % CPR;
  f16x8 g = {}, b = {};
  if (cy.mr_in) {
    g = *reinterpret_cast<const f16x8*>(rgb + c * 8);
    b = *reinterpret_cast<const f16x8*>(rgb + C::BN + c * 8);
  }
#pragma unroll kUnroll
  for (int q = 0; q < PER; ++q) {
    const int idx = threadIdx.x + q * C::THREADS;
    const int r = idx / CPR;
    if (idx < ROWS * CPR && m0 + r < M) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(tile + r * C::OUT_LD + c * 8);
      const size_t at = (size_t)(m0 + r) * N + n0 + c * 8;
      const f16x8 rv = ahead ? ahead->r[q] : *reinterpret_cast<const f16x8*>(residual + at);
      float y[8];
      if (cy.mr_in) {
        const float2 mr = rmr[r];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          y[i] = (float)v[i] + (((float)rv[i] - mr.x) * mr.y * (float)g[i] + (float)b[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = (float)v[i] + (float)rv[i];
      }
      f16x8 o;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        o[i] = (f16)y[i];
        y[i] = (float)o[i];  // the statistics describe the stored fp16 row
      }
      *reinterpret_cast<f16x8*>(out + at) = o;
      if (cy.st_out) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) t += y[i];
        t = xor_op<1>(t, AddOp{});
        t = xor_op<2>(t, AddOp{});
        t = xor_op<4>(t, AddOp{});
        const float mean = t * (1.0f / 64);
        float d2 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d2 += (y[i] - mean) * (y[i] - mean);
        d2 = xor_op<1>(d2, AddOp{});
        d2 = xor_op<2>(d2, AddOp{});
        d2 = xor_op<4>(d2, AddOp{});
        if ((c & 7) == 0)
          cy.st_out[(size_t)(m0 + r) * kMaxCarryTiles + (n0 + c * 8) / 64] = make_float2(mean, d2);
      }
    }
  }
}

// (mean, rstd) of a 384-wide row from the (mean, sum of squared deviations)
// pairs of its six 64-column groups (the pairwise update of Chan, Golub and
// LeVeque over all groups at once): the population variance the LayerNorm
// pass takes.
__device__ __forceinline__ float2 carried_row_stats(const float2 (&p)[kMaxCarryTiles], float eps) {
  float t = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxCarryTiles; ++k) t += p[k].x;
  const float mean = t * (1.0f / kMaxCarryTiles);
  float m2 = 0.f, d2 = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxCarryTiles; ++k) {
    const float d = p[k].x - mean;
    m2 += p[k].y;
    d2 += d * d;
  }
  m2 += d2 * 64.f;
  return make_float2(mean, rsqrtf(m2 * (1.0f / kHidden) + eps));
}

template <class C, int EPI>
__global__ __launch_bounds__(C::THREADS) void gemm_kernel(
    const f16* __restrict__ A, const f16* __restrict__ W, const f16* __restrict__ bias,
    const f16* residual, const f16* __restrict__ gamma, const f16* __restrict__ beta, f16* out,
    int M, int N, int K, float eps, LnCarry cy) {
  HIP_DYNAMIC_SHARED(f16, smem);
  int mi, ni;
  if (!tile_of(N / C::BN, (M + C::BM - 1) / C::BM, mi, ni)) return;
  const int m0 = mi * C::BM, n0 = ni * C::BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int r32 = lane & 31, kh = lane >> 5;

  // Per-column operands (bias; gamma and beta for LayerNorm) depend only on
  // the lane's columns.  Tiles with room in registers load them once, all
  // together, so their latency is paid once per tile instead of once per
  // 32x32 block; the 192-accumulator tiles load them once per column block.
  // Tiles with one or two 32-column blocks per wavefront and no LayerNorm
  // (8-16 VGPRs) load them before the K loop, as they do the residual, so
  // the loads' latency hides behind it.
  // The carried-LayerNorm GEMMs (kFold*) take fp32 fs / fc per column in
  // place of the bias, once per column block.
  constexpr bool kFoldE = EPI == kFold || EPI == kFoldGelu;
  constexpr bool kHoist = C::FM * C::FN <= 8 && !kFoldE;
  constexpr bool kColsAhead = kHoist && EPI != kLayerNorm && C::FN <= 2;
  constexpr int HN = kHoist ? C::FN : 1;
  f16x4 bvs[HN][4], gvs[EPI == kLayerNorm ? HN : 1][4], evs[EPI == kLayerNorm ? HN : 1][4];
  f32x4 fsv[kFoldE ? 4 : 1], fcv[kFoldE ? 4 : 1];
  // kFold*: fs / fc of the tile's columns in LDS after the row statistics
  // (written after the K loop; `fcol` is set there).
  const float* fcol = nullptr;
  auto load_cols = [&](int fn, int h) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nl = wn * C::TN + fn * 32 + 8 * j + 4 * kh;
      if constexpr (kFoldE) {
        fsv[j] = *reinterpret_cast<const f32x4*>(fcol + nl);
        fcv[j] = *reinterpret_cast<const f32x4*>(fcol + C::BN + nl);
      } else {
        bvs[h][j] = bias ? *reinterpret_cast<const f16x4*>(bias + n0 + nl) : f16x4{0, 0, 0, 0};
      }
      if constexpr (EPI == kLayerNorm) {
        gvs[h][j] = *reinterpret_cast<const f16x4*>(gamma + nl);
        evs[h][j] = *reinterpret_cast<const f16x4*>(beta + nl);
      }
    }
  };
  if constexpr (kColsAhead) {
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn) load_cols(fn, fn);
  }
  constexpr bool kAhead = (EPI == kResidual || EPI == kResStats) && ResidualAhead<C>::kOn;
  ResidualAhead<C> ahead;
  if constexpr (kAhead) ahead.load(residual, N, M, m0, n0);
  // kResStats with a carried residual: thread t < BM loads tile row t's
  // (mean, rstd), thread t < BN gamma / beta of tile column t; they go
  // through LDS to the store threads.  Before the K loop where the tile
  // keeps at most two residual chunks a thread in registers, after it
  // otherwise (the registers would cost the larger tiles occupancy).
  float2 smr = make_float2(0.f, 0.f);
  f16 sg = 0, sb = 0;
  auto load_carry = [&] {
    if (cy.mr_in) {
      if (threadIdx.x < C::BM) smr = cy.mr_in[min(m0 + (int)threadIdx.x, M - 1)];
      if (threadIdx.x < C::BN) {
        sg = gamma[n0 + threadIdx.x];
        sb = beta[n0 + threadIdx.x];
      }
    }
  };
  constexpr bool kCarryAhead = ResidualAhead<C>::PER <= 2;
  if constexpr (EPI == kResStats) {
    static_assert(C::THREADS >= C::BM && C::THREADS >= C::BN, "a thread per tile row / column");
    if constexpr (kCarryAhead) load_carry();
  }
  // kFold*: thread t < BM loads the six group pairs of tile row t (48
  // bytes), and thread t < BN fs / fc of tile column t, before the K loop,
  // so that their latency hides behind it.
  float2 rp[kFoldE ? kMaxCarryTiles : 1];
  float cs = 0.f, cc = 0.f;
  if constexpr (kFoldE) {
    static_assert(C::THREADS >= C::BM && C::THREADS >= C::BN, "a thread per tile row / column");
    if (threadIdx.x < C::BN) {
      cs = cy.fs[n0 + threadIdx.x];
      cc = cy.fc[n0 + threadIdx.x];
    }
    if (threadIdx.x < C::BM) {
      const f32x4* src = reinterpret_cast<const f32x4*>(
          cy.st_in + (size_t)min(m0 + (int)threadIdx.x, M - 1) * kMaxCarryTiles);
#pragma unroll
      for (int k = 0; k < kMaxCarryTiles / 2; ++k) {
        const f32x4 v = src[k];
        rp[2 * k] = make_float2(v[0], v[1]);
        rp[2 * k + 1] = make_float2(v[2], v[3]);
      }
    }
  }
  f32x16 acc[C::FM][C::FN];
  if constexpr (C::PD > 0)
    mainloop_reg<C>(A, W, M, K, m0, n0, smem, acc);
  else if constexpr (C::KPB > 1)
    mainloop_multi<C>(A, W, M, K, m0, n0, smem, acc);
  else
    mainloop<C>(A, W, M, K, m0, n0, smem, acc);

  constexpr int PR = C::BM / C::NPASS;  // tile rows staged per pass
  f16* tile = smem;                     // PR x OUT_LD fp16
  float* red = reinterpret_cast<float*>(smem + PR * C::OUT_LD);  // [2][WN][BM]
  float mean[C::FM], rstd[C::FM];
  if constexpr (kHoist && !kColsAhead) {
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn) load_cols(fn, fn);
  }
  float2* rmr = reinterpret_cast<float2*>(red);    // kResStats: [BM] (mean, rstd)
  f16* rgb = reinterpret_cast<f16*>(red + 2 * C::BM);  // kResStats: [2][BN] gamma, beta
  if constexpr (EPI == kResStats) {
    static_assert(C::RED >= (2 * C::BM) * sizeof(float) + 2 * C::BN * sizeof(f16),
                  "row statistics and gamma / beta fit the partials area");
    if constexpr (!kCarryAhead) load_carry();
    if (cy.mr_in) {  // read by the store threads after the tile pass's barrier
      if (threadIdx.x < C::BM) rmr[threadIdx.x] = smr;
      if (threadIdx.x < C::BN) {
        rgb[threadIdx.x] = sg;
        rgb[C::BN + threadIdx.x] = sb;
      }
    }
  }
  if constexpr (kFoldE) {
    // Each row's (mean, rstd) once, by its loader thread, into the LayerNorm
    // partials area (free for these epilogues), then to every lane of the
    // row; fs / fc after them.
    static_assert((size_t)(C::BM / C::NPASS) * C::OUT_LD * sizeof(f16) +
                          (2 * C::BM + 2 * C::BN) * sizeof(float) <= C::LDS,
                  "row statistics and column operands fit beside the output tile");
    float* fc_lds = red + 2 * C::BM;
    if (threadIdx.x < C::BM) {
      const float2 st = carried_row_stats(rp, eps);
      red[2 * threadIdx.x] = st.x;
      red[2 * threadIdx.x + 1] = st.y;
      const int m = m0 + (int)threadIdx.x;
      if (ni == 0 && m < M && cy.mr_out) cy.mr_out[m] = st;
    }
    if (threadIdx.x < C::BN) {
      fc_lds[threadIdx.x] = cs;
      fc_lds[C::BN + threadIdx.x] = cc;
    }
    fcol = fc_lds;
    lds_barrier();
#pragma unroll
    for (int fm = 0; fm < C::FM; ++fm) {
      const int row = wm * C::TM + fm * 32 + r32;
      mean[fm] = red[2 * row];
      rstd[fm] = red[2 * row + 1];
    }
  }

  if constexpr (EPI == kLayerNorm) {
    static_assert(C::BN == kHidden, "LayerNorm tile owns whole 384-wide rows");
    // v = acc + bias + residual, then the row statistics (lane ^ 32 holds the
    // other half of the wave's columns, LDS across wn).
    // The residual rows arrive through the (still free) output staging area:
    // coalesced 16-byte loads, then each lane reads its 4-column runs from
    // LDS.  Tiles staged in passes read their runs from global memory.
    // Staged residual: global_load_lds straight into LDS (no VGPRs while the
    // accumulators are live), unpadded [BM][384] with LDS chunk slot c of
    // row r holding logical chunk (c & ~7) | ((c ^ r) & 7).
    constexpr bool kStageRes = C::NPASS == 1;
    constexpr int kResCopies = C::BM * (kHidden / 8) / 64;  // 1 KB copies
    static_assert(!kStageRes || kResCopies % C::NW == 0, "residual copies per wavefront");
    auto res_at = [&](int r, int n) {  // halves offset of column n of staged row r
      const int c = n >> 3;
      return r * kHidden + (((c & ~7) | ((c ^ r) & 7)) << 3) + (n & 7);
    };
    if constexpr (kStageRes) {
#pragma unroll
      for (int j = 0; j < kResCopies / C::NW; ++j) {
        const int g = j * C::NW + wave;  // 1 KB copy index
        const int q = g * 64 + lane, r = q / (kHidden / 8), c = q % (kHidden / 8);
        const int cl = (c & ~7) | ((c ^ r) & 7);
        __builtin_amdgcn_global_load_lds(residual + (size_t)min(m0 + r, M - 1) * kHidden + cl * 8,
                                         (__attribute__((address_space(3))) void*)(tile + g * 512),
                                         16, 0, 0);
      }
      wait_vm<0>();
      lds_barrier();
    }
#pragma unroll
    for (int fn = 0; fn < C::FN; ++fn) {
      if constexpr (!kHoist) load_cols(fn, 0);
      const int h = kHoist ? fn : 0;
#pragma unroll
      for (int fm = 0; fm < C::FM; ++fm) {
        const int ml = wm * C::TM + fm * 32 + r32;
        const int mg = min(m0 + ml, M - 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n = wn * C::TN + fn * 32 + 8 * j + 4 * kh;
          const f16x4 rv =
              kStageRes ? *reinterpret_cast<const f16x4*>(tile + res_at(ml, n))
                        : *reinterpret_cast<const f16x4*>(residual + (size_t)mg * kHidden + n);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[fm][fn][4 * j + i] += (float)bvs[h][j][i] + (float)rv[i];
        }
      }
    }
    // Row statistics in one exchange: each wavefront's mean and squared
    // deviation over its TN columns of the row, combined across the WN
    // wavefronts of the row as equal-size groups (Chan et al.).
    float2* red2 = reinterpret_cast<float2*>(red);  // [WN][BM]
#pragma unroll
    for (int fm = 0; fm < C::FM; ++fm) {
      float s = 0.f;
#pragma unroll
      for (int fn = 0; fn < C::FN; ++fn)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += acc[fm][fn][i];
      const float mw = xor32_sum(s) * (1.0f / C::TN);
      float q = 0.f;
#pragma unroll
      for (int fn = 0; fn < C::FN; ++fn)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float d = acc[fm][fn][i] - mw;
          q += d * d;
        }
      q = xor32_sum(q);
      if (kh == 0) red2[wn * C::BM + wm * C::TM + fm * 32 + r32] = make_float2(mw, q);
    }
    lds_barrier();
#pragma unroll
    for (int fm = 0; fm < C::FM; ++fm) {
      const int row = wm * C::TM + fm * 32 + r32;
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < C::WN; ++w) t += red2[w * C::BM + row].x;
      mean[fm] = t * (1.0f / C::WN);
      float t2 = 0.f, dd = 0.f;
#pragma unroll
      for (int w = 0; w < C::WN; ++w) {
        const float2 pw = red2[w * C::BM + row];
        const float d = pw.x - mean[fm];
        t2 += pw.y;
        dd += d * d;
      }
      rstd[fm] = rsqrtf(fmaf((float)C::TN, dd, t2) * (1.0f / kHidden) + eps);
    }
  }

  // fp16 tile into LDS (row pass p holds tile rows [p*PR, (p+1)*PR)), then
  // coalesced stores, which add the residual for kResidual (16-byte loads laid
  // out like the output rows).  One 32x32 block at a time; the scheduling
  // fence keeps a single block's values live.
#pragma unroll
  for (int p = 0; p < C::NPASS; ++p) {
    if (C::NPASS == 1 || wm == p) {
#pragma unroll
      for (int fn = 0; fn < C::FN; ++fn) {
        if constexpr (!kHoist) load_cols(fn, 0);
        const int h = kHoist ? fn : 0;
#pragma unroll
        for (int fm = 0; fm < C::FM; ++fm) {
          const int ml = wm * C::TM + fm * 32 + r32;  // row inside the tile
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int nl = wn * C::TN + fn * 32 + 8 * j + 4 * kh;
            f16x4 o;
            if constexpr (EPI == kLayerNorm) {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                o[i] = to_half((acc[fm][fn][4 * j + i] - mean[fm]) * rstd[fm] *
                                   (float)gvs[h][j][i] +
                               (float)evs[h][j][i]);
            } else if constexpr (kFoldE) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                float v = fmaf(-mean[fm], fsv[j][i], acc[fm][fn][4 * j + i]) * rstd[fm] + fcv[j][i];
                if (EPI == kFoldGelu) v = gelu_poly(v);
                o[i] = to_half(v);
              }
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                float v = acc[fm][fn][4 * j + i] + (float)bvs[h][j][i];
                if (EPI == kGelu) v = gelu_poly(v);
                o[i] = to_half(v);
              }
            }
            *reinterpret_cast<f16x4*>(tile + (ml - p * PR) * C::OUT_LD + nl) = o;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    lds_barrier();
    if constexpr (EPI == kResStats)
      store_rows_stats<C, PR>(tile, out, M, m0 + p * PR, n0, residual, rmr + p * PR, rgb, cy,
                              kAhead ? &ahead : nullptr);
    else
      store_rows<C, PR>(tile, out, N, M, m0 + p * PR, n0, EPI == kResidual ? residual : nullptr,
                        kAhead ? ahead.r : nullptr);
    if (p + 1 < C::NPASS) lds_barrier();
  }
}

// ---- QKV Linear and attention in one kernel (forwards of up to 8192 rows) --
// A batch-64 forward spends about a tenth of its time in attention launches
// whose work is a few hundred cycles: one global round trip for Q, K and V
// just written by the QKV Linear, then the launch's tail.  Here workgroup
// (group of G = 128 / seq sentences, head h) computes the QKV Linear's 96
// columns of head h over the group's rows (a head-major copy of W: rows
// h*96 .. h*96+95 are Q, K, V of head h), with the bias or carried-LayerNorm
// epilogue of gemm_fold, writes them to LDS as Q rows, K rows (the attention
// kernel's swizzled layout) and V^T, and runs each sentence's masked
// attention from there, the arithmetic of attention_kernel with one query
// tile per wavefront: the same bits as the two kernels.
namespace qa {
constexpr int HD = kHeadDim, NQ = 3 * HD;
constexpr float kLazy = 8.f;  // as attention_kernel: the running max may lag by 2^8
// A workgroup of BM / 32 wavefronts over BM rows (128, or 192 where a
// sentence length fills it better).  LDS after the K loop (bytes): Q
// [BM][32], K [KR][32] (swizzled), V^T [32][VLD], key bias [G][round32(seq)]
// (at most 2 BM), row (mean, rstd) [BM], fs / fc [2][96], and each
// wavefront's 32 x 32 output tile [32][kOutLd] (all within the K loop's ring).
constexpr int kOutLd = 40;  // halves per row of a wavefront's output tile
template <int BM_>
struct Layout {
  static constexpr int BM = BM_, NWV = BM / 32, NT = 64 * NWV, KR = BM + 32, VLD = KR + 8;
  static constexpr int MBN = 2 * BM;  // >= G * round32(seq) for every seq, = NT
  using C = Cfg<BM, NQ, NWV, 1, 2, 0, 2>;
  static constexpr size_t OFF_Q = 0, OFF_K = OFF_Q + (size_t)BM * HD * 2,
                          OFF_V = OFF_K + (size_t)KR * HD * 2, OFF_B = OFF_V + (size_t)HD * VLD * 2,
                          OFF_R = OFF_B + (size_t)MBN * 4, OFF_F = OFF_R + (size_t)BM * 8,
                          OFF_S = (OFF_F + (size_t)2 * NQ * 4 + 15) & ~(size_t)15,
                          END = OFF_S + (size_t)NWV * 32 * kOutLd * 2;
  static constexpr size_t LDS = C::LDS > END ? C::LDS : END;
  static_assert(OFF_V % 16 == 0 && OFF_R % 16 == 0 && OFF_F % 16 == 0 && (VLD * 2) % 16 == 0,
                "align");
  static_assert(NT >= BM && NT >= NQ, "a thread per tile row / column");
};
// Rows a workgroup takes for a sentence length: 192 where 128 would leave a
// quarter or more of the tile idle (seq 48, 80, 96).
inline int rows_for(int seq) { return (seq == 48 || seq == 80 || seq == 96) ? 192 : 128; }
__device__ __forceinline__ int key_of_row(int r) {
  const int a = r >> 3, c = (r >> 2) & 1, b = r & 3;
  return 16 * (a >> 1) + 8 * c + 4 * (a & 1) + b;
}
__device__ __forceinline__ int ks_off(int key, int c) { return key * 32 + ((c ^ ((key >> 2) & 3)) << 3); }
}  // namespace qa

template <int BM_>
__global__ __launch_bounds__(2 * BM_) void qkv_attention_kernel(
    const f16* __restrict__ X, const f16* __restrict__ Wp, const float* __restrict__ fs,
    const float* __restrict__ fc, LnCarry cy, const int32_t* __restrict__ mask,
    f16* __restrict__ ctx, int batch, int seq, int G, float c, float eps) {
  using namespace qa;
  using L = Layout<BM_>;
  using C = typename L::C;
  constexpr int BM = L::BM, KR = L::KR, VLD = L::VLD, NT = L::NT;
  HIP_DYNAMIC_SHARED(f16, smem);
  const int x = blockIdx.x & 7, kx = blockIdx.x >> 3;
  const int grp = (kx / kHeads) * 8 + x, h = kx % kHeads;
  const int b0 = grp * G;
  if (b0 >= batch) return;  // the whole workgroup: no barrier reached
  const int gv = min(G, batch - b0), M = batch * seq, m0 = b0 * seq, R = gv * seq;
  const int ntq = (seq + 31) >> 5, KP = ntq * 32;  // query tiles (key chunks) per sentence
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r32 = lane & 31, kh = lane >> 5;

  // Before the K loop, so that their latency hides behind it: the six
  // group pairs of tile row tid (carried LayerNorm), fs / fc of column tid,
  // and the mask of (sentence tid / KP, key tid % KP).
  float2 rp[kMaxCarryTiles];
  if (cy.st_in && tid < BM) {
    const f32x4* src = reinterpret_cast<const f32x4*>(cy.st_in + (size_t)min(m0 + tid, M - 1) *
                                                                     kMaxCarryTiles);
#pragma unroll
    for (int k = 0; k < kMaxCarryTiles / 2; ++k) {
      const f32x4 v = src[k];
      rp[2 * k] = make_float2(v[0], v[1]);
      rp[2 * k + 1] = make_float2(v[2], v[3]);
    }
  }
  float cs = 0.f, cc = 0.f;
  if (tid < NQ) {
    cs = fs ? fs[h * NQ + tid] : 0.f;
    cc = fc[h * NQ + tid];
  }
  int mv = 0;
  if (tid < gv * KP) {
    const int g = tid / KP, key = tid - g * KP;
    if (key < seq) mv = mask[(size_t)(b0 + g) * seq + key];
  }

  f32x16 acc[1][3];
  mainloop<C>(X, Wp, M, kHidden, m0, h * NQ, smem, acc);

  unsigned char* lds = reinterpret_cast<unsigned char*>(smem);
  f16* Qs = reinterpret_cast<f16*>(lds + L::OFF_Q);
  f16* Ks = reinterpret_cast<f16*>(lds + L::OFF_K);
  f16* Vt = reinterpret_cast<f16*>(lds + L::OFF_V);
  float* mb = reinterpret_cast<float*>(lds + L::OFF_B);
  float2* rs = reinterpret_cast<float2*>(lds + L::OFF_R);
  float* fcol = reinterpret_cast<float*>(lds + L::OFF_F);
  if (tid < BM) {
    float2 st = make_float2(0.f, 1.f);  // no carried LayerNorm: acc + bias
    if (cy.st_in) {
      st = carried_row_stats(rp, eps);
      if (h == 0 && tid < R && cy.mr_out) cy.mr_out[m0 + tid] = st;
    }
    rs[tid] = st;
  }
  if (tid < NQ) {
    fcol[tid] = cs;
    fcol[NQ + tid] = cc;
  }
  if (tid < gv * KP) mb[tid] = mv != 0 ? 0.f : -INFINITY;
  // K rows and V^T columns BM .. KR-1, which a sentence's last key chunk may
  // reach past the group, hold zeros (their keys are masked).
  for (int i = tid; i < (KR - BM) * HD; i += NT) {
    Ks[BM * HD + i] = (f16)0.f;
    Vt[(i / (KR - BM)) * VLD + BM + i % (KR - BM)] = (f16)0.f;
  }
  lds_barrier();
  {
    // Epilogue: acc[0][fn][4j+e] is column fn*32 + 8j + 4kh + e (Q, K, V of
    // head h) of local row r, as gemm_fold computes it.
    const int r = wave * 32 + r32;
    const float2 st = rs[r];
#pragma unroll
    for (int fn = 0; fn < 3; ++fn)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 8 * j + 4 * kh;
        const f32x4 sv = *reinterpret_cast<const f32x4*>(fcol + fn * HD + d0);
        const f32x4 cv = *reinterpret_cast<const f32x4*>(fcol + NQ + fn * HD + d0);
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = to_half(fmaf(-st.x, sv[e], acc[0][fn][4 * j + e]) * st.y + cv[e]);
        if (fn == 0) {
          *reinterpret_cast<f16x4*>(Qs + r * HD + d0) = o;
        } else if (fn == 1) {
          *reinterpret_cast<f16x4*>(Ks + ks_off(r, j) + 4 * kh) = o;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) Vt[(d0 + e) * VLD + r] = o[e];
        }
      }
  }
  lds_barrier();

  // Attention: query tiles t0 .. t0 + T - 1 of sentence g (rows g*seq +
  // t*32 ..) per wavefront, over the sentence's key chunks.  T = 2 shares
  // each K and V^T operand read between a sentence's two tiles; each tile
  // keeps its own rescale decisions, so its bits are those of T = 1.
  const int krow = key_of_row(r32);
  const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const f16x2 ones = {(f16)1.f, (f16)1.f};
  const float lag = kLazy / c;
  f16* st = reinterpret_cast<f16*>(lds + L::OFF_S) + wave * 32 * kOutLd;
  auto attend = [&](auto Tc, int g, int t0) {
    constexpr int T = decltype(Tc)::value;
    const int kb = g * seq;
    f16x8 q0[T], q1[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      // Rows past the sentence read its last row (as attention_kernel clamps
      // them), so they take the same rescale decisions; they are not stored.
      const int qr = kb + min((t0 + t) * 32 + r32, seq - 1);
      q0[t] = *reinterpret_cast<const f16x8*>(Qs + qr * HD + 8 * kh);
      q1[t] = *reinterpret_cast<const f16x8*>(Qs + qr * HD + 16 + 8 * kh);
    }
    const float* mbg = mb + g * KP;
    f32x16 o[T];
    float m[T], l[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      o[t] = zero;
      m[t] = 0.f;
      l[t] = 0.f;
    }
    bool started = false;
    for (int kc = 0; kc < ntq; ++kc) {
      const uint32_t bits = (uint32_t)__ballot(mbg[kc * 32 + r32] == 0.f);
      if (bits == 0) continue;  // every key of the chunk masked: contributes nothing
      const int key = kb + kc * 32 + krow;
      const f16x8 k0 = *reinterpret_cast<const f16x8*>(Ks + ks_off(key, kh));
      const f16x8 k1 = *reinterpret_cast<const f16x8*>(Ks + ks_off(key, 2 + kh));
      f32x16 sc[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        sc[t] = mfma32(k0, q0[t], zero);
        sc[t] = mfma32(k1, q1[t], sc[t]);  // sc[i]: key kc*32 + 16*(i/8) + 8*kh + i%8 (raw)
      }
      if (bits != 0xffffffffu) {
        const float* mk = mbg + kc * 32 + 8 * kh;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float bias = mk[16 * (i >> 3) + (i & 7)];
#pragma unroll
          for (int t = 0; t < T; ++t) sc[t][i] += bias;
        }
      }
      float mx[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        float v = __builtin_elementwise_maximum(__builtin_elementwise_maximum(sc[t][0], sc[t][1]),
                                                sc[t][2]);
#pragma unroll
        for (int i = 3; i < 15; i += 2)
          v = __builtin_elementwise_maximum(__builtin_elementwise_maximum(v, sc[t][i]), sc[t][i + 1]);
        v = __builtin_elementwise_maximum(v, sc[t][15]);
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                         false, false);
        mx[t] = __builtin_elementwise_maximum(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      if (!started) {
#pragma unroll
        for (int t = 0; t < T; ++t) m[t] = mx[t];
        started = true;
      } else {
#pragma unroll
        for (int t = 0; t < T; ++t)
          if (__ballot(mx[t] > m[t] + lag)) {
            const float mn = fmaxf(m[t], mx[t]);
            const float corr = __builtin_amdgcn_exp2f((m[t] - mn) * c);
            l[t] *= corr;
            o[t] *= corr;
            m[t] = mn;
          }
      }
      const f16* vrow = Vt + r32 * VLD + kb + kc * 32 + 8 * kh;
      const f16x8 va = *reinterpret_cast<const f16x8*>(vrow);
      const f16x8 vb = *reinterpret_cast<const f16x8*>(vrow + 16);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float mc = m[t] * c;
        f16x8 pa, pb;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pa[i] = (f16)__builtin_amdgcn_exp2f(fmaf(sc[t][i], c, -mc));
          pb[i] = (f16)__builtin_amdgcn_exp2f(fmaf(sc[t][8 + i], c, -mc));
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
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float lt = xor32_sum(l[t]);
      const float inv = lt > 0.f ? 1.0f / lt : 0.f;
      // Out through this wavefront's own LDS tile (o[i] = O[tile row r32]
      // [8*(i/4) + 4*kh + i%4]), so that each store writes 16 query rows x 64
      // contiguous bytes; the wavefront's LDS accesses stay in order, so no
      // barrier (also between its tiles).
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (f16)(o[t][4 * j + e] * inv);
        *reinterpret_cast<f16x4*>(st + r32 * kOutLd + 8 * j + 4 * kh) = w;
      }
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int row = 16 * p + (lane >> 2), cc = lane & 3, q = (t0 + t) * 32 + row;
        const f16x8 w = *reinterpret_cast<const f16x8*>(st + row * kOutLd + 8 * cc);
        if (q < seq)
          *reinterpret_cast<f16x8*>(ctx + (size_t)(m0 + kb + q) * kHidden + h * HD + 8 * cc) = w;
      }
    }
  };
  // Two-tile sentences (seq 33 .. 64) a wavefront each where one tile per
  // wavefront would take two rounds (seq 48 on 192 rows: 8 tiles, 6
  // wavefronts); otherwise one tile per wavefront.
  // Seq 16: two sentences a 32-row tile (queries and keys 0-15 of sentence
  // g0, 16-31 of g0 + 1) with the cross-sentence pairs masked, so half the
  // tiles.  A query's probabilities and sums are those of its own sentence's
  // tile: the other sentence's keys give exact zeros in the same MFMA and
  // fdot2 positions its padding keys held there.
  if (seq == 16) {
    for (int pr = wave; 2 * pr < gv; pr += L::NWV) {
      const int g0 = 2 * pr, kb = g0 * 16, qs = r32 >> 4;  // this lane's query: sentence g0 + qs
      const int qr = min(kb + r32, R - 1);
      const f16x8 q0 = *reinterpret_cast<const f16x8*>(Qs + qr * HD + 8 * kh);
      const f16x8 q1 = *reinterpret_cast<const f16x8*>(Qs + qr * HD + 16 + 8 * kh);
      const int key = kb + krow;
      const f16x8 k0 = *reinterpret_cast<const f16x8*>(Ks + ks_off(key, kh));
      const f16x8 k1 = *reinterpret_cast<const f16x8*>(Ks + ks_off(key, 2 + kh));
      f32x16 sc = mfma32(k0, q0, zero);
      sc = mfma32(k1, q1, sc);  // sc[i]: key 16*(i/8) + 8*kh + i%8 of the tile, sentence g0 + i/8
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int ks = i >> 3;
        sc[i] += (ks == qs && g0 + ks < gv) ? mb[(g0 + ks) * KP + 8 * kh + (i & 7)] : -INFINITY;
      }
      float v = __builtin_elementwise_maximum(__builtin_elementwise_maximum(sc[0], sc[1]), sc[2]);
#pragma unroll
      for (int i = 3; i < 15; i += 2)
        v = __builtin_elementwise_maximum(__builtin_elementwise_maximum(v, sc[i]), sc[i + 1]);
      v = __builtin_elementwise_maximum(v, sc[15]);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                       false, false);
      const float mx = __builtin_elementwise_maximum(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      // every key of the query's sentence masked: zero context, as a skipped chunk gives
      const float mc = (mx == -INFINITY ? 0.f : mx) * c;
      const f16* vrow = Vt + r32 * VLD + kb + 8 * kh;
      const f16x8 va = *reinterpret_cast<const f16x8*>(vrow);
      const f16x8 vb = *reinterpret_cast<const f16x8*>(vrow + 16);
      f16x8 pa, pb;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pa[i] = (f16)__builtin_amdgcn_exp2f(fmaf(sc[i], c, -mc));
        pb[i] = (f16)__builtin_amdgcn_exp2f(fmaf(sc[8 + i], c, -mc));
      }
      float l = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        l = __builtin_amdgcn_fdot2(f16x2{pa[i], pa[i + 1]}, ones, l, false);
        l = __builtin_amdgcn_fdot2(f16x2{pb[i], pb[i + 1]}, ones, l, false);
      }
      f32x16 o = mfma32(va, pa, zero);
      o = mfma32(vb, pb, o);
      const float lt = xor32_sum(l);
      const float inv = lt > 0.f ? 1.0f / lt : 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (f16)(o[4 * j + e] * inv);
        *reinterpret_cast<f16x4*>(st + r32 * kOutLd + 8 * j + 4 * kh) = w;
      }
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int row = 16 * p + (lane >> 2), cc = lane & 3;
        const f16x8 w = *reinterpret_cast<const f16x8*>(st + row * kOutLd + 8 * cc);
        if (kb + row < R)
          *reinterpret_cast<f16x8*>(ctx + (size_t)(m0 + kb + row) * kHidden + h * HD + 8 * cc) = w;
      }
    }
  } else if (ntq == 2 && 2 * gv > L::NWV) {
    for (int g = wave; g < gv; g += L::NWV) attend(std::integral_constant<int, 2>{}, g, 0);
  } else {
    for (int qt = wave; qt < gv * ntq; qt += L::NWV)
      attend(std::integral_constant<int, 1>{}, qt / ntq, qt % ntq);
  }
}

// ---- Weight-resident kernel for K = 384 -----------------------------------
// The QKV and FFN1 Linears have K = 384, so one wavefront can hold the fp16 W
// fragments of 32 output columns for the whole K in 96 VGPRs.  A workgroup of
// 12 wavefronts (768 threads, 3 per SIMD) then owns 384 columns and walks
// 32-row M-tiles persistently.  W arrives once, in the prologue, through LDS
// (contiguous 1 KB copies, then fragment reads): per-lane 16-byte loads of 32
// rows at a time ran at ~15 B/clk per CU and left ~8 us of every launch
// before the first MFMA.  Only A streams through LDS after that: a ring of
// wres::RING tiles of 32 x 384 (24 KB each, the 64-wide slice layout above),
// filled with global_load_lds, two 1 KB copies per wavefront per tile.  No W
// moves after the prologue, and each 32x32x16 MFMA reads one 1 KB A fragment
// from LDS.  Bytes moved from L2 per FLOP drop ~6x against a 128x128 tile;
// on MI355X that delivery, not the matrix cores, bounds the tiled kernels.
//
// The k order, operand layout, epilogue arithmetic and fp16 rounding are
// those of the tiled kernels, so every output is bit-identical whichever
// kernel computes it.
namespace wres {
constexpr int NW = 12, THREADS = 64 * NW, K = 384, KS = K / 16, BM = 32, RING = 4;
constexpr int TILE = BM * K;                   // halves per A tile
constexpr int CPW = (BM * K * 2 / 1024) / NW;  // 1 KB copies per wavefront per tile
constexpr int COLS = NW * 32;                  // output columns per workgroup
constexpr int kStageLd = 40;  // halves per row of a wavefront's 32 x 32 output block
// A ring, per-wavefront output staging, LayerNorm row partials [2][NW][32].
constexpr size_t LDS =
    ((size_t)RING * TILE + (size_t)NW * 32 * kStageLd) * sizeof(f16) + 2 * NW * 32 * sizeof(float);
// The LayerNorm epilogue also holds the tile's residual rows ([BM][K], 16-byte
// chunks swizzled within groups of 8) and the bias, gamma and beta of the
// workgroup's columns.
constexpr size_t LDS_LN = LDS + ((size_t)BM * K + 3 * (size_t)COLS) * sizeof(f16);
static_assert(LDS_LN <= kLdsMax, "LDS");
static_assert((BM * K * 2 / 1024) % NW == 0 && BM * K * 2 / 1024 == 2 * NW, "copies per wavefront");
}  // namespace wres

template <int EPI>
__global__ __launch_bounds__(wres::THREADS) void gemm_wres_kernel(
    const f16* __restrict__ A, const f16* __restrict__ W, const f16* __restrict__ bias,
    f16* out, int M, int N, const f16* residual = nullptr, const f16* __restrict__ gamma = nullptr,
    const f16* __restrict__ beta = nullptr, float eps = 0.f) {
  using namespace wres;
  HIP_DYNAMIC_SHARED(f16, smem);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r32 = lane & 31, kh = lane >> 5;
  // Workgroup b runs on XCD b % 8.  The nb column blocks of one M-group are
  // placed on the same XCD, so each A tile comes from HBM once per XCD.
  const int nb = N / COLS, x = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int ng = slot % nb, mg = (slot / nb) * 8 + x, groups = (int)(gridDim.x >> 3) / nb * 8;
  const int n0 = ng * COLS + wave * 32;
  // W fragment of k-step s: row n0 + r32, k = 16 s + 8 kh .. +7 (the tiled
  // kernels' k mapping).
  f16x8 w[KS];
  {
    // The workgroup's 384 W rows (contiguous, 768 B each) come through LDS in
    // rounds of RR rows, two LDS buffers in turn so that the copies of round
    // r + 1 are in flight while round r is read: contiguous 1 KB
    // global_load_lds copies, then each of the round's wavefronts reads its
    // 32 rows' fragments.  In LDS, 16-byte chunk c of row r sits at slot
    // c ^ (r & 15) of the row, so the 16 rows of one fragment read fall on
    // distinct banks.
    constexpr int CH = K * 2 / 16;            // 48 chunks per row
    constexpr int RR = 64;                    // rows per round (32: no faster)
    constexpr int NR = COLS / RR;             // rounds
    constexpr int CPR = RR * CH / (64 * NW);  // copies per wavefront per round
    constexpr int BUF = RR * K;               // halves per buffer
    static_assert(RR * CH % (64 * NW) == 0 && (size_t)2 * BUF * 2 <= LDS && RR % 32 == 0,
                  "W rounds");
    const f16* Wb = W + (size_t)ng * COLS * K;
    auto copy_round = [&](int rd) {
      f16* buf = smem + (rd & 1) * BUF;
#pragma unroll
      for (int j = 0; j < CPR; ++j) {
        const int p = (j * NW + wave) * 64 + lane, row = p / CH, slot = p % CH;
        __builtin_amdgcn_global_load_lds(
            Wb + (size_t)(rd * RR + row) * K + (slot ^ (row & 15)) * 8,
            (__attribute__((address_space(3))) void*)(buf + (j * NW + wave) * 512), 16, 0, 0);
      }
    };
    copy_round(0);
#pragma unroll 1
    for (int rd = 0; rd < NR; ++rd) {
      if (rd + 1 < NR) {
        copy_round(rd + 1);  // its buffer was last read in round rd - 1
        wait_vm<CPR>();      // round rd landed (copies retire in issue order)
      } else {
        wait_vm<0>();
      }
      lds_barrier();
      if (wave / (RR / 32) == rd) {
        const f16* buf = smem + (rd & 1) * BUF;
        const int row = (wave % (RR / 32)) * 32 + r32;
#pragma unroll
        for (int st = 0; st < KS; ++st)
          w[st] = *reinterpret_cast<const f16x8*>(buf + row * K + 8 * ((2 * st + kh) ^ (row & 15)));
      }
      lds_barrier();  // buffer rd & 1 is refilled by round rd + 2 (or the A ring)
    }
  }
  // Bias of this lane's 16 columns, held for the whole kernel (the LayerNorm
  // epilogue re-reads it per tile instead: its registers are spoken for).
  f16x4 bq[4];
  auto load_bias = [&] {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bq[j] = bias ? *reinterpret_cast<const f16x4*>(bias + n0 + 8 * j + 4 * kh) : f16x4{0, 0, 0, 0};
  };
  if (EPI != kLayerNorm) load_bias();
  // LayerNorm: bias | gamma | beta of the 384 columns once into LDS, so no
  // global load sits in the tile loop.  The compiler's wait for a global load
  // there is vmcnt(0), which would drain every A copy in flight each tile.
  f16* resid = smem + RING * TILE + NW * 32 * kStageLd + 4 * NW * 32;  // after the partials
  f16* colv = resid + BM * K;
  if constexpr (EPI == kLayerNorm) {
    for (int q = threadIdx.x; q < 3 * COLS / 8; q += THREADS) {
      const int v = q / (COLS / 8), c = q % (COLS / 8);
      const f16* src = v == 0 ? bias : v == 1 ? gamma : beta;
      const f16x8 x = src ? *reinterpret_cast<const f16x8*>(src + ng * COLS + 8 * c)
                          : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      *reinterpret_cast<f16x8*>(colv + v * COLS + 8 * c) = x;
    }
  }
  const int ntiles = (M + BM - 1) / BM;
  const int my = mg < ntiles ? (ntiles - 1 - mg) / groups + 1 : 0;
  // Copy g of a tile: slice g / 4, rows (g % 4) * 8 .. +7 (copy_group's lane
  // layout); rows past M read row M - 1.
  auto issue = [&](int i) {
    const int t = mg + i * groups;
    f16* dst = smem + (i % RING) * TILE;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const int g = wave * CPW + j, sl = g >> 2, r = (g & 3) * 8 + (lane >> 3);
      const int cl = (lane & 7) ^ Slice<64>::f(r);
      __builtin_amdgcn_global_load_lds(
          A + (size_t)min(t * BM + r, M - 1) * K + sl * 64 + cl * 8,
          (__attribute__((address_space(3))) void*)(dst + sl * 2048 + (g & 3) * 512), 16, 0, 0);
    }
  };
  // LayerNorm: tile i's residual rows (rows past M read row M - 1) into LDS.
  // Each wavefront copies exactly the part it reads back, its own 32
  // columns (16-byte chunks 4 wave .. 4 wave + 3) of the 32 rows, so that it
  // waits for its own copies only, with no barrier: copy j2 (1 KB) holds rows
  // 16 j2 .. +15, lane l row 16 j2 + l / 4 in slot l % 4, which holds
  // logical chunk (l % 4) ^ ((row >> 2) & 3) (the 16 rows of one read fall on
  // distinct banks).
  auto issue_res = [&](int i) {
    const int t = mg + i * groups;
#pragma unroll
    for (int j2 = 0; j2 < 2; ++j2) {
      const int r = 16 * j2 + (lane >> 2), c = 4 * wave + ((lane & 3) ^ ((r >> 2) & 3));
      __builtin_amdgcn_global_load_lds(
          residual + (size_t)min(t * BM + r, M - 1) * K + c * 8,
          (__attribute__((address_space(3))) void*)(resid + (j2 * NW + wave) * 512), 16, 0, 0);
    }
  };
#pragma unroll
  for (int i = 0; i < RING - 1; ++i)
    if (i < my) issue(i);
  for (int i = 0; i < my; ++i) {
    // Tile i has landed once at most the loads issued after its copies are
    // outstanding (loads retire in issue order among themselves; the
    // epilogue stores, also counted in vmcnt, only make the wait stricter):
    // the copies of tiles i+1 .. i+RING-2, and with LayerNorm also the
    // residual copies of tiles i-2 and i-1 (issued after tile i's from i = 2).
    if constexpr (EPI == kLayerNorm) {
      if (i >= 2 && i + RING - 2 < my)
        wait_vm<CPW * (RING - 2) + 4>();
      else
        wait_vm<0>();
    } else {
      if (i + RING - 2 < my)
        wait_vm<CPW * (RING - 2)>();
      else
        wait_vm<0>();
    }
    lds_barrier();  // tile i visible to all; tile i-1's slot (and residual) free
    if constexpr (EPI == kLayerNorm) issue_res(i);
    if (i + RING - 1 < my) issue(i + RING - 1);
    const f16* tA = smem + (i % RING) * TILE;
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    f16x8 a[2];
    a[0] = *reinterpret_cast<const f16x8*>(tA + Slice<64>::off(r32, kh));
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      if (st + 1 < KS) {
        const int s1 = st + 1;
        a[s1 & 1] = *reinterpret_cast<const f16x8*>(tA + (s1 >> 2) * 2048 +
                                                     Slice<64>::off(r32, 2 * (s1 & 3) + kh));
      }
      acc = mfma32(w[st], a[st & 1], acc);
    }
    // acc[i] = D(n0 + 8 (i / 4) + 4 kh + i % 4, m): four 4-column runs of row m.
    const int m0 = (mg + i * groups) * BM;
    f16* stg = smem + RING * TILE + wave * 32 * kStageLd;
    if constexpr (EPI == kLayerNorm) {
      // N = 384: the workgroup owns whole rows.  v = acc + bias + residual,
      // then the row statistics in one exchange: each wavefront's mean and
      // squared deviation over its 32 columns (a lane's 16, lane ^ 32 holds
      // the other 16), combined across the 12 wavefronts as equal-size
      // groups (Chan et al.).  A wavefront reads only the residual elements
      // it then overwrites, so out may alias residual.
      float2* red = reinterpret_cast<float2*>(smem + RING * TILE + NW * 32 * kStageLd);  // [NW][32]
      // This wavefront's residual copies of the tile: only those of tile
      // i+RING-1 were issued after them.
      if (i + RING - 1 < my)
        wait_vm<CPW>();
      else
        wait_vm<0>();
      const f16* cv = colv + wave * 32 + 4 * kh;
#pragma unroll
      for (int j = 0; j < 4; ++j) bq[j] = *reinterpret_cast<const f16x4*>(cv + 8 * j);
      const f16* rrow = resid + ((r32 >> 4) * NW + wave) * 512 + (r32 & 15) * 32 + 4 * kh;
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // columns wave * 32 + 8 j + 4 kh .. +3
        const f16x4 rv = *reinterpret_cast<const f16x4*>(rrow + ((j ^ ((r32 >> 2) & 3)) << 3));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * j + e] += (float)bq[j][e] + (float)rv[e];
      }
      float sm = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) sm += acc[e];
      const float mw = xor32_sum(sm) * (1.0f / 32);
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float d = acc[e] - mw;
        q += d * d;
      }
      q = xor32_sum(q);
      if (kh == 0) red[wave * 32 + r32] = make_float2(mw, q);
      lds_barrier();
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += red[w * 32 + r32].x;
      const float mean = t * (1.0f / NW);
      float t2 = 0.f, dd = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {  // read again: registers are short here
        const float2 pw = red[w * 32 + r32];
        const float d = pw.x - mean;
        t2 += pw.y;
        dd += d * d;
      }
      const float rstd = rsqrtf(fmaf(32.f, dd, t2) * (1.0f / kHidden) + eps);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f16x4 g = *reinterpret_cast<const f16x4*>(cv + COLS + 8 * j);
        const f16x4 be = *reinterpret_cast<const f16x4*>(cv + 2 * COLS + 8 * j);
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = to_half((acc[4 * j + e] - mean) * rstd * (float)g[e] + (float)be[e]);
        *reinterpret_cast<f16x4*>(stg + r32 * kStageLd + 8 * j + 4 * kh) = o;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = acc[4 * j + e] + (float)bq[j][e];
          if (EPI == kGelu) v = gelu_poly(v);
          o[e] = to_half(v);
        }
        *reinterpret_cast<f16x4*>(stg + r32 * kStageLd + 8 * j + 4 * kh) = o;
      }
    }
    // Back out of this wavefront's own LDS block (no barrier needed) as
    // 16-byte stores, each instruction 16 rows x 64 contiguous bytes: 1.5-2x
    // the HBM write rate of the 8-byte stores straight from the accumulator
    // layout (32 rows x 16 bytes per instruction).
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int row = 16 * p + (lane >> 2), cc = lane & 3;
      const f16x8 v = *reinterpret_cast<const f16x8*>(stg + row * kStageLd + 8 * cc);
      if (m0 + row < M)
        *reinterpret_cast<f16x8*>(out + (size_t)(m0 + row) * N + n0 + 8 * cc) = v;
    }
  }
}

// The weight-resident kernel serves K = 384 and N a multiple of 384, from
// the M where sweeps on MI355X show it ahead of the tiled kernels: 16384 for
// FFN1 (N = 1536, where it saves the most L2 traffic per row), 24576 for QKV.
bool wres_ok(int M, int N, int K) {
  return K == wres::K && N % wres::COLS == 0 && M >= (N >= 1536 ? 16384 : 24576);
}

template <int EPI>
hipError_t launch_wres(const f16* A, const f16* W, const f16* bias, f16* out, int M, int N,
                       hipStream_t s, const f16* residual = nullptr, const f16* gamma = nullptr,
                       const f16* beta = nullptr, float eps = 0.f) {
  if (EPI == kLayerNorm && N != wres::COLS) return hipErrorInvalidValue;
  constexpr size_t lds = EPI == kLayerNorm ? wres::LDS_LN : wres::LDS;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_wres_kernel<EPI>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  // One workgroup per CU: 8 XCDs x nb column blocks x q M-groups per XCD.
  const int nb = N / wres::COLS, ntiles = (M + wres::BM - 1) / wres::BM;
  const int q = max(1, min(cus / (8 * nb), (ntiles + 7) / 8));
  hipLaunchKernelGGL((gemm_wres_kernel<EPI>), dim3(8 * nb * q), dim3(wres::THREADS), lds, s,
                     A, W, bias, out, M, N, residual, gamma, beta, eps);
  return hipGetLastError();
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

template <class C, int EPI>
hipError_t launch(const f16* A, const f16* W, const f16* bias, const f16* residual,
                  const f16* gamma, const f16* beta, f16* out, int M, int N, int K, float eps,
                  hipStream_t s, const LnCarry& cy = LnCarry{}) {
  if constexpr (EPI == kLayerNorm && C::BN != kHidden) {
    return hipErrorInvalidValue;  // LayerNorm needs a tile that owns whole rows
  } else if constexpr (EPI == kResStats && C::BN != 64 && C::BN != 128) {
    return hipErrorInvalidValue;  // row statistics over 8 or 16 lanes
  } else {
    if (N % C::BN != 0) return hipErrorInvalidValue;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_kernel<C, EPI>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
    if (attr != hipSuccess) return attr;
    // Row chunks of at most 2^30 bytes of A each: the K loop addresses A
    // through 32-bit buffer offsets.
    const int step = std::max(C::BM, (int)((1 << 30) / ((size_t)K * 2)) / C::BM * C::BM);
    if ((size_t)N * K * 2 >= (1u << 31)) return hipErrorInvalidValue;
    for (int r0 = 0; r0 < M; r0 += step) {
      const int mr = std::min(step, M - r0);
      const int nb = N / C::BN, mb = (mr + C::BM - 1) / C::BM;
      const int grid = nb * 8 * ((mb + 7) / 8);
      LnCarry cr = cy;  // row-indexed like A and out
      if (cr.st_in) cr.st_in += (size_t)r0 * kMaxCarryTiles;
      if (cr.mr_out) cr.mr_out += r0;
      if (cr.mr_in) cr.mr_in += r0;
      if (cr.st_out) cr.st_out += (size_t)r0 * kMaxCarryTiles;
      hipLaunchKernelGGL((gemm_kernel<C, EPI>), dim3(grid), dim3(C::THREADS), C::LDS, s,
                         A + (size_t)r0 * K, W, bias, residual ? residual + (size_t)r0 * N : nullptr,
                         gamma, beta, out + (size_t)r0 * N, mr, N, K, eps, cr);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
}

// Tile configurations (BM, BN, wavefronts M x N, A-ring depth), by id; the K
// slice is 64 wide and the W ring 2 deep but in tile 34.  The product build holds
// the configurations pick_plain and gemm_residual_ln_tile choose; the others
// of the sweep that chose them are compiled only with -DBBH_TUNING.
//   id  tile      wave tile  SA   LDS
//    0  64x64     32x32      4    48 KB
//    1  64x128    32x64      4    64 KB
//   14  64x384    64x96      2   112 KB   (owns whole 384-wide rows)
//   8 wavefronts (2 per SIMD):
//   18  128x384   64x96      4   160 KB   (owns whole rows)
//   19  256x192   64x96      3   144 KB
//   register-staged K slices (PD slices in flight in VGPRs, LDS double buffer):
//   26  64x64     32x32      PD 4   32 KB
//   28  128x384   64x96 (8w) PD 2  128 KB   (owns whole rows)
//   30  128x128   64x32 (8w) PD 2   64 KB
//   31  128x128   32x64 (8w) PD 2   64 KB
//   32  128x192   32x96 (8w) PD 2   80 KB
//   copy rings with two K slices per barrier (PD -2; A and W rings 4 deep):
//   34  64x64     32x32      4/4    64 KB
// Kernel symbols read gemm_kernel<Cfg<BM,BN,WM,WN,SA,PD,SW>, epilogue>.
// The table itself: X(id, BM, BN, WM, WN, SA, PD, SW).
#define BBH_TILES(X) \
  X(0, 64, 64, 2, 2, 4, 0, 2) \
  X(1, 64, 128, 2, 2, 4, 0, 2) \
  X(14, 64, 384, 1, 4, 2, 0, 2) \
  X(18, 128, 384, 2, 4, 4, 0, 2) \
  X(19, 256, 192, 4, 2, 3, 0, 2) \
  X(26, 64, 64, 2, 2, 2, 4, 2) \
  X(28, 128, 384, 2, 4, 2, 2, 2) \
  X(30, 128, 128, 2, 4, 2, 2, 2) \
  X(31, 128, 128, 4, 2, 2, 2, 2) \
  X(32, 128, 192, 4, 2, 2, 2, 2) \
  X(34, 64, 64, 2, 2, 4, -2, 4)

#ifdef BBH_TUNING
// The rest of the sweep (ids 2-13, 15-17, 20-25, 27, 29).
#define BBH_TUNING_TILES(X) \
  X(2, 128, 64, 2, 2, 4, 0, 2) \
  X(3, 128, 128, 2, 2, 4, 0, 2) \
  X(4, 256, 128, 2, 2, 3, 0, 2) \
  X(5, 128, 384, 1, 4, 4, 0, 2) \
  X(6, 64, 384, 1, 4, 4, 0, 2) \
  X(7, 32, 128, 1, 4, 4, 0, 2) \
  X(8, 128, 192, 2, 2, 4, 0, 2) \
  X(9, 256, 192, 2, 2, 3, 0, 2) \
  X(10, 32, 384, 1, 4, 4, 0, 2) \
  X(11, 128, 384, 1, 4, 3, 0, 2) \
  X(12, 256, 192, 2, 2, 2, 0, 2) \
  X(13, 128, 192, 2, 2, 3, 0, 2) \
  X(15, 128, 128, 2, 2, 2, 0, 2) \
  X(16, 64, 128, 2, 2, 6, 0, 2) \
  X(17, 256, 384, 2, 4, 2, 0, 2) \
  X(20, 256, 128, 4, 2, 3, 0, 2) \
  X(21, 128, 256, 2, 4, 4, 0, 2) \
  X(22, 128, 128, 2, 2, 2, 3, 2) \
  X(23, 128, 128, 2, 2, 2, 4, 2) \
  X(24, 128, 256, 2, 4, 2, 2, 2) \
  X(25, 256, 128, 4, 2, 2, 2, 2) \
  X(27, 128, 192, 2, 2, 2, 3, 2) \
  X(29, 256, 128, 2, 2, 2, 3, 2)
#else
#define BBH_TUNING_TILES(X)
#endif

constexpr int kTiles = 33;  // kTiles names the weight-resident kernel (no tile has this id)

// The Cfg of a product tile id.
template <int ID>
struct TileOf;
#define BBH_TILE_TYPE(ID, BM, BN, WM, WN, SA, PD, SW) \
  template <>                                         \
  struct TileOf<ID> {                                 \
    using type = Cfg<BM, BN, WM, WN, SA, PD, SW>;     \
  };
BBH_TILES(BBH_TILE_TYPE)
#undef BBH_TILE_TYPE
template <int ID>
using TileCfg = typename TileOf<ID>::type;

template <int EPI>
hipError_t launch_id(int id, const f16* A, const f16* W, const f16* bias, const f16* residual,
                     const f16* gamma, const f16* beta, f16* out, int M, int N, int K, float eps,
                     hipStream_t s) {
#define BBH_CASE(ID, BM, BN, WM, WN, SA, PD, SW)                                     \
  case ID:                                                                           \
    return launch<Cfg<BM, BN, WM, WN, SA, PD, SW>, EPI>(A, W, bias, residual, gamma, \
                                                        beta, out, M, N, K, eps, s);
  switch (id) {
    BBH_TILES(BBH_CASE)
    BBH_TUNING_TILES(BBH_CASE)
  }
#undef BBH_CASE
  return hipErrorInvalidValue;
}

int bn_of(int id) {
#define BBH_BN(ID, BM, BN, WM, WN, SA, PD, SW) \
  case ID:                                     \
    return BN;
  switch (id) {
    BBH_TILES(BBH_BN)
    BBH_TUNING_TILES(BBH_BN)
  }
#undef BBH_BN
  return 0;
}

const char* tile_name(int id) {
#define BBH_NAME(ID, BM, BN, WM, WN, SA, PD, SW) \
  case ID:                                       \
    return "Cfg<" #BM "," #BN "," #WM "," #WN "," #SA "," #PD "," #SW ">";
  switch (id) {
    BBH_TILES(BBH_NAME)
    BBH_TUNING_TILES(BBH_NAME)
  }
#undef BBH_NAME
  return nullptr;
}

// Tile config per shape, from interleaved A/B timings (medians of several
// rounds) on MI355X over the encoder's four shapes (N, K) = (1152, 384) QKV,
// (1536, 384) FFN1, (384, 384) O-proj and (384, 1536) FFN2.  QKV and FFN1 at
// large M run on the weight-resident kernel instead (wres_ok).  Small M wants
// many small tiles (latency, CU coverage); large M wants big tiles (L2 and
// LDS traffic per MFMA).  Up to 4096 rows (the batch-64 forwards of the
// length buckets) the best tile depends on whether other forwards share the
// CUs.
// Alone (shared false: bbh_embed, a one-slot pool), from sweeps of the
// configs[1] and one-slot configs[3] forwards with one GEMM's tile changed at
// a time: QKV runs the 64x64 copy-ring tile (0) up to 1024 rows (configs[1]
// forward 230.1 -> 224.3 us: 288 workgroups instead of 72); FFN1 keeps that
// tile to 4096 rows (with the LayerNorm carried in: one-slot pass 8.22-8.24
// -> 8.11 ms against the register-staged 64x64 at 2049-3072 rows); O-proj
// and FFN2 from 2049 rows run the 64x64 copy ring with two K slices per
// barrier (34; one-slot varlen pass 9.00-9.03 -> 8.84-8.95 ms).  More
// workgroups than CUs keep every CU busy, and the deeper rings fit beside
// nothing else.  At 513-1024 rows alone FFN1 takes tile 34 (configs[1]
// forward 195.4-195.8 -> 194.6-194.8 us, four interleaved repeats); at
// 6145-8192 rows alone FFN1 takes tile 31, FFN2 tile 30 and O-proj tile 0
// (configs[2] forward 387.5 -> 383.5 us on one box, every repeat; level on
// a slower one).
// Beside other forwards (shared true: a pool of several slots) every tile was
// tried for each (shape, M) with the others fixed in the per-batch pass, then
// the winners confirmed in interleaved repeats: FFN1 takes the 128x128
// register-staged tile (30) from 1025 rows and FFN2 the 64x128 copy-ring tile
// (1) from 2049 rows, 391K -> 409K sentences/s for the pass on three streams.
// With the LayerNorms carried as row statistics (the epilogues heavier), a
// sweep on four slots moved O-proj to tile 1 as well and QKV to tile 30 up to
// 4096 rows: pass 4.144-4.160 -> 4.064-4.095 ms in four interleaved repeats;
// with QKV inside the attention kernel, O-proj to the 128x128 tile (30):
// 4.117-4.127 -> 4.092-4.104 ms; FFN2 on tile 1 and O-proj on tile 30 from
// 1025 rows as well (3.708 -> 3.668 ms, then 3.845-3.857 -> 3.828-3.843 ms,
// four repeats each; alone they are slower there).
// There the other forwards fill the CUs, and fewer, larger tiles move fewer
// bytes L2 -> CU per FLOP.
int pick_plain(int M, int N, int K, bool shared) {
  const bool qkv = N == 1152, ffn1 = N == 1536, wide_k = K >= 1024;
  int id;
  if (M <= 1024)
    id = qkv ? (shared ? 30 : 0) : ffn1 ? (!shared && M > 512 ? 34 : 0) : 26;
  else if (M <= 2048)
    id = qkv ? 30 : ffn1 ? (shared ? 30 : 0) : !shared ? 26 : wide_k ? 1 : 30;
  else if (M <= 3072)
    id = qkv ? 30 : ffn1 ? (shared ? 30 : 0) : !shared ? 34 : wide_k ? 1 : 30;
  else if (M <= 4096)
    id = qkv ? (shared ? 30 : 32) : ffn1 ? (shared ? 30 : 0) : !shared ? 34 : wide_k ? 1 : 30;
  else if (M <= 6144)
    id = qkv ? 30 : ffn1 ? 26 : wide_k ? 31 : 0;
  else if (M <= 8192)
    id = shared ? (wide_k ? 31 : 30) : qkv ? 30 : ffn1 ? 31 : wide_k ? 30 : 0;
  else if (M <= 16384)
    id = wide_k ? 32 : 30;
  else if (M <= 49152)
    id = wide_k ? 19 : 30;
  else
    id = qkv ? 19 : ffn1 ? 31 : wide_k ? 19 : 30;
  return (N % bn_of(id) == 0) ? id : 0;  // id 0 takes any N % 64 == 0
}

}  // namespace

bool gemm_mfma_ok(int N, int K) { return N % 64 == 0 && K % 64 == 0; }

int gemm_tile(int M, int N, int K, bool shared) {
  if (!gemm_mfma_ok(N, K)) return -1;
  return wres_ok(M, N, K) ? kTiles : pick_plain(M, N, K, shared);
}

// Large M: one kernel whose 128x384 tile owns whole rows.  Smaller M: a tile
// that owns whole rows leaves most CUs idle and streams all of W per
// workgroup, so the GEMM runs on 2-D tiles with a bias + residual epilogue
// (in place over y) and the row LayerNorm follows as its own pass.
// The weight-resident kernel takes the K = 384 LayerNorm Linear (O-proj)
// from M = 65536, where it passes tile 28 (89.5 vs 98.0 us at M = 131072;
// at M = 26857 its fixed W prologue leaves it 15% behind).
int gemm_residual_ln_tile(int M, int K, bool* fused_ln, bool shared) {
  *fused_ln = M > 8192;
  if (!*fused_ln) return pick_plain(M, kHidden, K, shared);
  if (K == wres::K && M >= 65536) return kTiles;
  return M <= 16384 ? 14 : K >= 1024 ? 18 : 28;
}

const char* gemm_tile_name(int tile) {
  if (tile == kTiles) return "WRes<12x32,384>";
  const char* n = tile_name(tile);
  return n ? n : "generic";
}

hipError_t gemm(const f16* A, const f16* W, const f16* bias, f16* C, int M, int N, int K,
                Act act, hipStream_t s, bool shared) {
  const bool gelu = act == Act::kGelu;
  const bool aligned = (((uintptr_t)A | (uintptr_t)W | (uintptr_t)C) & 15) == 0 &&
                       ((uintptr_t)bias & 7) == 0;
  if (!gemm_mfma_ok(N, K) || !aligned) {
    dim3 grid((N + 15) / 16, (M + 15) / 16);
    hipLaunchKernelGGL(gemm_generic_kernel, grid, dim3(256), 0, s, A, W, bias, C, M, N, K,
                       gelu ? 1 : 0);
    return hipGetLastError();
  }
  if (wres_ok(M, N, K))
    return gelu ? launch_wres<kGelu>(A, W, bias, C, M, N, s) : launch_wres<kBias>(A, W, bias, C, M, N, s);
  const int id = pick_plain(M, N, K, shared);
  return gelu ? launch_id<kGelu>(id, A, W, bias, nullptr, nullptr, nullptr, C, M, N, K, 0.f, s)
              : launch_id<kBias>(id, A, W, bias, nullptr, nullptr, nullptr, C, M, N, K, 0.f, s);
}

hipError_t gemm_residual_ln(const f16* A, const f16* W, const f16* bias, const f16* residual,
                            const f16* gamma, const f16* beta, f16* y, int M, int K, float eps,
                            hipStream_t s, bool shared) {
  bool fused;
  const int id = gemm_residual_ln_tile(M, K, &fused, shared);
  if (id == kTiles)
    return launch_wres<kLayerNorm>(A, W, bias, y, M, kHidden, s, residual, gamma, beta, eps);
  if (fused)
    return launch_id<kLayerNorm>(id, A, W, bias, residual, gamma, beta, y, M, kHidden, K, eps, s);
  hipError_t e = gemm_residual(A, W, bias, residual, y, M, K, s, shared);
  if (e != hipSuccess) return e;
  return layernorm(y, nullptr, gamma, beta, y, M, kHidden, eps, s);
}

// The carried-LayerNorm epilogues are built for the tiles pick_plain chooses
// up to 8192 rows.
template <int EPI>
hipError_t launch_carry(int id, const f16* A, const f16* W, const f16* bias, const f16* residual,
                        const f16* gamma, const f16* beta, f16* out, int M, int N, int K, float eps,
                        hipStream_t s, const LnCarry& cy) {
#define BBH_CARRY(ID)                                                                          \
  case ID:                                                                                     \
    return launch<TileCfg<ID>, EPI>(A, W, bias, residual, gamma, beta, out, M, N, K, eps, s, cy);
  switch (id) {
    BBH_CARRY(0)
    BBH_CARRY(1)
    BBH_CARRY(26)
    BBH_CARRY(30)
    BBH_CARRY(31)
    BBH_CARRY(32)
    BBH_CARRY(34)
  }
#undef BBH_CARRY
  return hipErrorInvalidValue;
}

bool ln_carry_ok(int M) { return M >= 1 && M <= 8192; }

template <int BM>
hipError_t launch_qkv_attention(const f16* X, const f16* Wp, const float* fs, const float* fc,
                                const LnCarry& cy, const int32_t* mask, f16* ctx, int batch, int seq,
                                float c, float eps, hipStream_t s) {
  using L = qa::Layout<BM>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(qkv_attention_kernel<BM>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)L::LDS);
  if (attr != hipSuccess) return attr;
  const int G = BM / seq, groups = (batch + G - 1) / G;
  const int grid = kHeads * 8 * ((groups + 7) / 8);
  hipLaunchKernelGGL(qkv_attention_kernel<BM>, dim3(grid), dim3(L::NT), L::LDS, s, X, Wp, fs, fc, cy,
                     mask, ctx, batch, seq, G, c, eps);
  return hipGetLastError();
}

bool qkv_attention_ok(int batch, int seq) {
  return batch >= 1 && seq >= 16 && seq <= 128 && seq % 16 == 0 && ln_carry_ok(batch * seq);
}

hipError_t qkv_attention(const f16* X, const f16* Wp, const float* fs, const float* fc,
                         const LnCarry& cy, const int32_t* mask, f16* ctx, int batch, int seq,
                         float scale, float eps, hipStream_t s) {
  const bool aligned = (((uintptr_t)X | (uintptr_t)Wp | (uintptr_t)ctx) & 15) == 0 &&
                       (((uintptr_t)cy.st_in) & 15) == 0;
  if (!qkv_attention_ok(batch, seq) || !fc || !mask || !aligned) return hipErrorInvalidValue;
  const float c = scale * 1.4426950408889634f;  // scores * c are base-2 exponents
  return qa::rows_for(seq) == 192
             ? launch_qkv_attention<192>(X, Wp, fs, fc, cy, mask, ctx, batch, seq, c, eps, s)
             : launch_qkv_attention<128>(X, Wp, fs, fc, cy, mask, ctx, batch, seq, c, eps, s);
}

hipError_t gemm_fold(const f16* A, const f16* W, const LnCarry& cy, f16* C, int M, int N, int K,
                     Act act, float eps, hipStream_t s, bool shared) {
  const bool aligned = (((uintptr_t)A | (uintptr_t)W | (uintptr_t)C) & 15) == 0 &&
                       (((uintptr_t)cy.fs | (uintptr_t)cy.fc) & 15) == 0;
  if (!ln_carry_ok(M) || !gemm_mfma_ok(N, K) || !aligned || !cy.st_in || !cy.fs || !cy.fc ||
      wres_ok(M, N, K))
    return hipErrorInvalidValue;
  const int id = pick_plain(M, N, K, shared);
  return act == Act::kGelu
             ? launch_carry<kFoldGelu>(id, A, W, nullptr, nullptr, nullptr, nullptr, C, M, N, K, eps, s, cy)
             : launch_carry<kFold>(id, A, W, nullptr, nullptr, nullptr, nullptr, C, M, N, K, eps, s, cy);
}

hipError_t gemm_residual_stats(const f16* A, const f16* W, const f16* bias, const f16* residual,
                               const f16* gamma, const f16* beta, const LnCarry& cy, f16* y,
                               int M, int K, hipStream_t s, bool shared) {
  bool fused;
  const int id = gemm_residual_ln_tile(M, K, &fused, shared);
  if (fused || !ln_carry_ok(M) || (cy.mr_in && (!gamma || !beta))) return hipErrorInvalidValue;
  return launch_carry<kResStats>(id, A, W, bias, residual, gamma, beta, y, M, kHidden, K, 0.f, s,
                                 cy);
}

hipError_t gemm_residual(const f16* A, const f16* W, const f16* bias, const f16* residual, f16* y,
                         int M, int K, hipStream_t s, bool shared) {
  bool fused;
  const int id = gemm_residual_ln_tile(M, K, &fused, shared);
  if (fused) return hipErrorInvalidValue;
  return launch_id<kResidual>(id, A, W, bias, residual, nullptr, nullptr, y, M, kHidden, K, 0.f, s);
}

#ifdef BBH_TUNING
// Tuning hook (built only with -DBBH_TUNING): run tile config `id` with
// epilogue epi (0 bias, 1 gelu, 2 residual, 3 layernorm).
extern "C" int bbh_tune_gemm(int id, int epi, const void* A, const void* W, const void* bias,
                             const void* residual, const void* gamma, const void* beta, void* out,
                             int M, int N, int K, float eps, void* stream) {
  auto a = static_cast<const f16*>(A);
  auto w = static_cast<const f16*>(W);
  auto b = static_cast<const f16*>(bias);
  auto r = static_cast<const f16*>(residual);
  auto g = static_cast<const f16*>(gamma);
  auto be = static_cast<const f16*>(beta);
  auto o = static_cast<f16*>(out);
  auto st = static_cast<hipStream_t>(stream);
  if (id == kTiles) {  // the weight-resident kernel, any M
    if (K != wres::K || N % wres::COLS != 0 || epi == 2) return hipErrorInvalidValue;
    if (epi == 3) return launch_wres<kLayerNorm>(a, w, b, o, M, N, st, r, g, be, eps);
    return epi ? launch_wres<kGelu>(a, w, b, o, M, N, st) : launch_wres<kBias>(a, w, b, o, M, N, st);
  }
  switch (epi) {
    case 0: return launch_id<kBias>(id, a, w, b, r, g, be, o, M, N, K, eps, st);
    case 1: return launch_id<kGelu>(id, a, w, b, r, g, be, o, M, N, K, eps, st);
    case 2: return launch_id<kResidual>(id, a, w, b, r, g, be, o, M, N, K, eps, st);
    case 3: return launch_id<kLayerNorm>(id, a, w, b, r, g, be, o, M, N, K, eps, st);
  }
  return hipErrorInvalidValue;
}
#endif

}  // namespace bbh

// Host launchers of the gfx950 kernels.  Each enqueues on `s` and returns the
// launch status; argument validation happens in capi.cpp before these run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace bbh {

enum class Act { kNone, kGelu };

// One sentence of a packed forward: its `len` valid tokens (the leading ones
// of its padded row, ids/types at tok .. tok + len - 1) occupy hidden rows
// row .. row + len - 1, and its embedding goes to row out_row of the output.
struct PackedSentence {
  int64_t tok, out_row;
  int32_t row, len;
};

// C(M,N) = A(M,K) . W(N,K)^T [+ bias] [GELU].  True when the MFMA path takes
// the shape (N % 64 == 0, K % 64 == 0); otherwise the plain tiled kernel runs.
// `shared` (here and below): other forwards run beside this one on the GPU
// (a pool of several slots), which changes the best tile from 1025 to 4096
// rows; the result is the same either way.
bool gemm_mfma_ok(int N, int K);
hipError_t gemm(const f16* A, const f16* W, const f16* bias, f16* C, int M, int N,
                int K, Act act, hipStream_t s, bool shared = false);

// The encoder's LayerNorms carried between its GEMMs as row statistics
// instead of passes of their own, where the residual GEMM tiles do not own
// whole rows (M <= 8192, ln_carry_ok).  A residual GEMM (gemm_residual_stats)
// writes y = A . W^T + bias + R un-normalised, and for each row the mean and
// the sum of squared deviations of its fp16 outputs over each of its six
// 64-column groups (st_out: kMaxCarryTiles pairs a row, the same bits
// whatever the tile).  R is the residual as given, or, with
// mr_in, the residual rows brought through their LayerNorm on the fly from
// each row's (mean, rstd).  The GEMM that reads y (gemm_fold: QKV, FFN1)
// combines a row's pairs into its mean and rstd, writes those (mr_out, by the
// workgroups of the first column tile) for the next residual GEMM, and gives
// LN(y) . W^T + bias as rstd * (y . W'^T - mean * fs) + fc, W' = W diag(gamma)
// in fp16, fs = row sums of W', fc = W . beta + bias (fp32, per column).
struct LnCarry {
  const float2* st_in = nullptr;  // gemm_fold: the input rows' group pairs
  float2* mr_out = nullptr;       // gemm_fold: (mean, rstd) per row
  const float* fs = nullptr;      // gemm_fold: per output column
  const float* fc = nullptr;
  const float2* mr_in = nullptr;  // gemm_residual_stats: (mean, rstd) of the residual rows
  float2* st_out = nullptr;       // gemm_residual_stats: the output rows' group pairs
};
constexpr int kMaxCarryTiles = 6;  // 64-column groups of a 384-wide row
bool ln_carry_ok(int M);
hipError_t gemm_fold(const f16* A, const f16* W, const LnCarry& cy, f16* C, int M, int N, int K,
                     Act act, float eps, hipStream_t s, bool shared = false);
hipError_t gemm_residual_stats(const f16* A, const f16* W, const f16* bias, const f16* residual,
                               const f16* gamma, const f16* beta, const LnCarry& cy, f16* y,
                               int M, int K, hipStream_t s, bool shared = false);

// The QKV Linear and masked attention of a padded batch in one kernel
// (qkv_attention_ok: seq a multiple of 16 up to 128, batch*seq <= 8192):
// ctx (merged heads) from the hidden rows X.  Wp is the QKV weight in
// head-major row order (rows h*96 .. h*96+95: Q, K, V of head h), fs / fc
// per column in the same order; the epilogue is gemm_fold's with the input
// rows' statistics from cy (st_in, and mr_out written) or, without st_in,
// acc + fc (fc the bias).  The same bits as that Linear and attention().
bool qkv_attention_ok(int batch, int seq);
hipError_t qkv_attention(const f16* X, const f16* Wp, const float* fs, const float* fc,
                         const LnCarry& cy, const int32_t* mask, f16* ctx, int batch, int seq,
                         float scale, float eps, hipStream_t s);

// Tile configuration gemm() / gemm_residual_ln() launch for a shape (-1: the
// plain tiled kernel), whether the LayerNorm is inside the GEMM kernel, and
// the configuration's name as it appears in the kernel symbol.
int gemm_tile(int M, int N, int K, bool shared = false);
int gemm_residual_ln_tile(int M, int K, bool* fused_ln, bool shared = false);
const char* gemm_tile_name(int tile);

// y(M,384) = LN(A(M,K) . W(384,K)^T + bias + residual) * gamma + beta.
// y may alias residual.  K % 64 == 0.
hipError_t gemm_residual_ln(const f16* A, const f16* W, const f16* bias,
                            const f16* residual, const f16* gamma, const f16* beta,
                            f16* y, int M, int K, float eps, hipStream_t s,
                            bool shared = false);

// The first half of gemm_residual_ln where gemm_residual_ln_tile says the
// LayerNorm is not fused: y = A . W^T + bias + residual (fp16), which a
// layernorm(y, ...) pass then normalises in place.
hipError_t gemm_residual(const f16* A, const f16* W, const f16* bias, const f16* residual, f16* y,
                         int M, int K, hipStream_t s, bool shared = false);

// The whole feed-forward block in one kernel for M >= ffn_fused_ok's bound:
// out(M,384) = LN(GELU(X . W1^T + b1) . W2^T + b2 + X) * gamma + beta, with the
// intermediate kept on chip; the arithmetic of gemm(.., kGelu) followed by
// gemm_residual_ln (equal but for rare fp16 rounding midpoints).  out may
// alias X.  X, W1, W2, out 16-byte aligned; the vectors 8-byte aligned.
bool ffn_fused_ok(int M);
hipError_t ffn_fused(const f16* X, const f16* W1, const f16* b1, const f16* W2, const f16* b2,
                     const f16* gamma, const f16* beta, f16* out, int M, float eps, hipStream_t s);

// Fused masked attention from the QKV activations (row stride 3*heads*32).
hipError_t attention(const f16* qkv, const int32_t* mask, f16* merged, int batch,
                     int heads, int seq, float scale, hipStream_t s);

// The same over packed sentences (no padding rows, no mask): workgroup (s, h)
// attends over rows sents[s].row .. + len.  max_len bounds every len.
hipError_t attention_packed(const f16* qkv, const PackedSentence* sents, int n, f16* merged,
                            int heads, int max_len, float scale, hipStream_t s);

// Reference-shaped attention pieces (unfused): scores, masked softmax, context.
hipError_t attention_scores(const f16* qkv, f16* scores, int batch, int heads, int seq,
                            int qkv_stride, int q_off, int k_off, float scale,
                            hipStream_t s);
hipError_t softmax_rows(f16* x, int M, int N, const int32_t* mask, int mask_stride,
                        hipStream_t s);
hipError_t attention_context(const f16* probs, const f16* qkv, f16* merged, int batch,
                             int heads, int seq, int qkv_stride, int v_off,
                             hipStream_t s);

// Row LayerNorm of (x [+ residual]); y may alias x or residual.
hipError_t layernorm(const f16* x, const f16* residual, const f16* gamma,
                     const f16* beta, f16* y, int M, int D, float eps, hipStream_t s);

// Embedding gather-sum, plain and fused with the embedding LayerNorm.
hipError_t embedding(const int32_t* ids, const int32_t* types, const f16* word,
                     const f16* pos, const f16* type, f16* out, int batch, int seq,
                     int hidden, hipStream_t s);
hipError_t embedding_ln(const int32_t* ids, const int32_t* types, const f16* word,
                        const f16* pos, const f16* type, const f16* gamma,
                        const f16* beta, f16* out, int batch, int seq, float eps,
                        hipStream_t s);

// Embedding + LayerNorm and mean pool + L2 normalise over packed sentences
// (one workgroup per sentence).
hipError_t embedding_ln_packed(const int32_t* ids, const int32_t* types, const f16* word,
                               const f16* pos, const f16* type, const f16* gamma,
                               const f16* beta, f16* out, const PackedSentence* sents, int n,
                               float eps, hipStream_t s);
hipError_t pool_normalize_packed(const f16* hidden, const PackedSentence* sents, int n,
                                 f16* out, hipStream_t s);

// Masked mean pool, L2 normalise, and the two fused.
hipError_t mean_pool(const f16* hidden, const int32_t* mask, f16* out, int batch,
                     int seq, int dim, hipStream_t s);
hipError_t l2_normalize(f16* x, int n, int batch, hipStream_t s);
hipError_t pool_normalize(const f16* hidden, const int32_t* mask, f16* out, int batch,
                          int seq, hipStream_t s);
// LayerNorm (gamma, beta, eps) of each counted row of y, then pool_normalize:
// equal to layernorm(y) followed by pool_normalize; y is left as it was.
hipError_t ln_pool_normalize(const f16* y, const int32_t* mask, const f16* gamma,
                             const f16* beta, float eps, f16* out, int batch, int seq,
                             hipStream_t s);

// Exact-erf GELU in place over n values.
hipError_t gelu(f16* x, size_t n, hipStream_t s);

}  // namespace bbh

// C ABI of the engine (include/bbh.h): weight loading, workspace, forward
// orchestration, argument validation and error reporting.
//
// Forward per encoder layer (the reference's attention_block + ffn_block,
// src/model/encoder.cu:25-71, with 9 launches per layer) is 5 launches here:
//   1. QKV GEMM + bias                       hidden   -> qkv      (M, 1152)
//   2. fused masked attention                qkv      -> ctx      (M, 384)
//   3. O GEMM + bias + residual(hidden) + LN ctx      -> attn_out (M, 384)
//   4. FFN1 GEMM + bias + GELU               attn_out -> inter    (M, 1536)
//   5. FFN2 GEMM + bias + residual + LN      inter    -> out      (M, 384)
// plus one fused embedding+LN launch before the layers and one fused
// pool+normalize launch after them: 32 launches per bert_embed against the
// reference's 58 launches and a device-to-device copy (src/model/forward.cu).

#include <ctype.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <math.h>

#include <string>
#include <algorithm>
#include <map>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/bbh.h"
#include "kernels.h"

using bbh::f16;

namespace {

thread_local std::string g_err;

bbh_status fail(bbh_status s, const std::string& msg) {
  g_err = msg;
  return s;
}

}  // namespace

// The thread's last-error message, for the library's other host sources
// (tokenizer.cpp).
namespace bbh_detail {
bbh_status set_error(bbh_status s, const std::string& msg) { return fail(s, msg); }
}  // namespace bbh_detail

namespace {

bbh_status hip_fail(hipError_t e, const char* what) {
  return fail(BBH_ERR_HIP, std::string(what) + ": " + hipGetErrorName(e) + " (" +
                               hipGetErrorString(e) + ")");
}

#define BBH_HIP(call, what)                           \
  do {                                                \
    hipError_t _e = (call);                           \
    if (_e != hipSuccess) return hip_fail(_e, what);  \
  } while (0)

struct Param {
  std::string name;
  size_t numel;
  size_t rows = 0;  // 2-D tensors: the (out) row count; 0 for vectors
};

const std::vector<Param>& params() {
  static const std::vector<Param> p = [] {
    std::vector<Param> v;
    const size_t H = BBH_HIDDEN, F = BBH_FFN_DIM;
    v.push_back({"embeddings.word_embeddings.weight", (size_t)BBH_VOCAB_SIZE * H, BBH_VOCAB_SIZE});
    v.push_back({"embeddings.position_embeddings.weight", (size_t)BBH_MAX_POSITION * H,
                 BBH_MAX_POSITION});
    v.push_back({"embeddings.token_type_embeddings.weight", (size_t)BBH_TYPE_VOCAB_SIZE * H,
                 BBH_TYPE_VOCAB_SIZE});
    v.push_back({"embeddings.LayerNorm.weight", H});
    v.push_back({"embeddings.LayerNorm.bias", H});
    for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
      const std::string p = "encoder.layer." + std::to_string(i) + ".";
      for (const char* part : {"query", "key", "value"}) {
        v.push_back({p + "attention.self." + part + ".weight", H * H, H});
        v.push_back({p + "attention.self." + part + ".bias", H});
      }
      v.push_back({p + "attention.output.dense.weight", H * H, H});
      v.push_back({p + "attention.output.dense.bias", H});
      v.push_back({p + "attention.output.LayerNorm.weight", H});
      v.push_back({p + "attention.output.LayerNorm.bias", H});
      v.push_back({p + "intermediate.dense.weight", F * H, F});
      v.push_back({p + "intermediate.dense.bias", F});
      v.push_back({p + "output.dense.weight", H * F, H});
      v.push_back({p + "output.dense.bias", H});
      v.push_back({p + "output.LayerNorm.weight", H});
      v.push_back({p + "output.LayerNorm.bias", H});
    }
    return v;
  }();
  return p;
}

constexpr int kPerLayer = 16;  // state_dict tensors per encoder layer
constexpr int kEmbParams = 5;

constexpr size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Forwards of up to kCarryMaxRows rows carry their LayerNorms as row
// statistics (bbh::ln_carry_ok); a workspace holds those statistics for
// min(rows, kCarryMaxRows) rows: two buffers of tile pairs, two of
// (mean, rstd).
constexpr size_t kCarryMaxRows = 8192;
constexpr size_t carry_rows(size_t rows) { return std::min(rows, kCarryMaxRows); }
constexpr size_t carry_bytes(size_t rows) {
  const size_t rc = carry_rows(rows);
  return 2 * align256(rc * bbh::kMaxCarryTiles * sizeof(float2)) + 2 * align256(rc * sizeof(float2));
}

}  // namespace

struct bbh_model {
  void* blob = nullptr;
  size_t bytes = 0;
  void* fold_blob = nullptr;  // the carried-LayerNorm operands (fold_operands)
  size_t fold_bytes = 0;
  const f16 *word, *pos, *type, *emb_g, *emb_b;
  struct Layer {
    const f16 *qkv_w, *qkv_b, *o_w, *o_b, *ln1_g, *ln1_b;
    const f16 *f1_w, *f1_b, *f2_w, *f2_b, *ln2_g, *ln2_b;
    // The GEMMs that read rows whose LayerNorm is carried as statistics
    // (bbh::LnCarry): QKV from layer 1 (the previous layer's ln2) and FFN1
    // (this layer's ln1): W' = W diag(gamma) (W itself when gamma is all
    // ones), fs = row sums of W', fc = W . beta + bias.
    const f16 *qkv_wf = nullptr, *f1_wf = nullptr;
    const float *qkv_fs = nullptr, *qkv_fc = nullptr, *f1_fs = nullptr, *f1_fc = nullptr;
    // The QKV Linear of bbh::qkv_attention: qkv_wf (or qkv_w in layer 0) in
    // head-major row order, its fs (none in layer 0) and fc (the bias in
    // layer 0) in the same order.
    const f16* qkv_wp = nullptr;
    const float *qkv_fsp = nullptr, *qkv_fcp = nullptr;
  } layers[BBH_NUM_LAYERS];
};

struct bbh_workspace {
  int max_batch = 0, max_seq = 0;
  size_t rows = 0;
  void* blob = nullptr;
  size_t bytes = 0;
  f16 *qkv, *ctx, *attn_out, *inter, *ping, *pong;
  // Carried LayerNorms (forwards of at most carry_rows rows): tile pairs and
  // (mean, rstd) of the attention block's (a) and the FFN block's (b) rows.
  float2 *st_a = nullptr, *st_b = nullptr, *mr_a = nullptr, *mr_b = nullptr;
  size_t carry_rows = 0;
  bbh::PackedSentence* sents;  // plan of a packed forward: up to `rows` sentences
  bool shared = false;         // a slot of a multi-slot pool: other forwards run beside
};

namespace {

// Device blob layout: the five embedding tensors, then per layer
// qkv_w (1152x384, Q|K|V rows), qkv_b, o_w, o_b, ln1 g/b, f1_w, f1_b, f2_w,
// f2_b, ln2 g/b; every array starts on a 256-byte boundary.
struct BlobLayout {
  std::vector<size_t> off;  // offset (elements) of each state_dict tensor in the blob
  size_t total = 0;         // elements
};

const BlobLayout& layout() {
  static const BlobLayout L = [] {
    BlobLayout l;
    const auto& p = params();
    l.off.assign(p.size(), 0);
    size_t cur = 0;  // bytes
    auto put = [&](int idx) {
      l.off[idx] = cur / sizeof(f16);
      cur = align256(cur + p[idx].numel * sizeof(f16));
    };
    for (int i = 0; i < kEmbParams; ++i) put(i);
    for (int L_ = 0; L_ < BBH_NUM_LAYERS; ++L_) {
      const int b0 = kEmbParams + L_ * kPerLayer;
      // Q|K|V weights contiguous (fused 1152x384), then Q|K|V biases contiguous.
      const size_t H = BBH_HIDDEN;
      l.off[b0 + 0] = cur / 2;
      l.off[b0 + 2] = cur / 2 + H * H;
      l.off[b0 + 4] = cur / 2 + 2 * H * H;
      cur = align256(cur + 3 * H * H * 2);
      l.off[b0 + 1] = cur / 2;
      l.off[b0 + 3] = cur / 2 + H;
      l.off[b0 + 5] = cur / 2 + 2 * H;
      cur = align256(cur + 3 * H * 2);
      for (int k = 6; k < kPerLayer; ++k) put(b0 + k);
    }
    l.total = cur / sizeof(f16);
    return l;
  }();
  return L;
}

float f16_bits_to_float(uint16_t b) {
  f16 h;
  memcpy(&h, &b, sizeof h);
  return (float)h;
}

// The carried-LayerNorm operands of every layer (bbh_model::Layer), from the
// host copy of the weights, into one device allocation: fs and fc in fp32
// (sums in double), W' = fp16(W * gamma) (the fp32 product of two fp16
// values is exact, so one rounding) only where gamma is not all ones.
bbh_status fold_operands(const std::vector<uint16_t>& host, bbh_model* m) {
  const BlobLayout& L = layout();
  const size_t H = BBH_HIDDEN;
  struct Fold {
    int layer, w, b, g, be;  // param indices: W (N x 384), bias, gamma, beta
    size_t n;
    bool qkv;
  };
  std::vector<Fold> folds;
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    const int b0 = kEmbParams + i * kPerLayer;
    if (i > 0) {
      const int p0 = kEmbParams + (i - 1) * kPerLayer;
      folds.push_back({i, b0 + 0, b0 + 1, p0 + 14, p0 + 15, 3 * H, true});
    }
    folds.push_back({i, b0 + 10, b0 + 11, b0 + 8, b0 + 9, (size_t)BBH_FFN_DIM, false});
  }
  // layout: per fold fs | fc (fp32), then W' where needed
  std::vector<size_t> vec_at(folds.size()), w_at(folds.size(), SIZE_MAX);
  std::vector<bool> ones(folds.size());
  size_t cur = 0;
  for (size_t f = 0; f < folds.size(); ++f) {
    vec_at[f] = cur;
    cur = align256(cur + 2 * folds[f].n * sizeof(float));
  }
  for (size_t f = 0; f < folds.size(); ++f) {
    const uint16_t* g = host.data() + L.off[folds[f].g];
    bool all = true;
    for (size_t k = 0; k < H; ++k) all = all && g[k] == 0x3C00;  // fp16 1.0
    ones[f] = all;
    if (!all) {
      w_at[f] = cur;
      cur = align256(cur + folds[f].n * H * sizeof(f16));
    }
  }
  // Head-major QKV operands per layer: W (row h*96 + part*32 + d from row
  // part*384 + h*32 + d), fs, fc.
  std::vector<size_t> hm_at(BBH_NUM_LAYERS);
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    hm_at[i] = cur;
    cur = align256(cur + 3 * H * H * sizeof(f16));
    cur = align256(cur + 2 * 3 * H * sizeof(float));
  }
  std::vector<unsigned char> buf(cur, 0);
  for (size_t f = 0; f < folds.size(); ++f) {
    const Fold& fd = folds[f];
    const uint16_t* W = host.data() + L.off[fd.w];
    const uint16_t* bias = host.data() + L.off[fd.b];
    const uint16_t* g = host.data() + L.off[fd.g];
    const uint16_t* be = host.data() + L.off[fd.be];
    float* fs = reinterpret_cast<float*>(buf.data() + vec_at[f]);
    float* fc = fs + fd.n;
    f16* wf = ones[f] ? nullptr : reinterpret_cast<f16*>(buf.data() + w_at[f]);
    for (size_t n = 0; n < fd.n; ++n) {
      double ss = 0.0, cc = 0.0;
      for (size_t k = 0; k < H; ++k) {
        const float w = f16_bits_to_float(W[n * H + k]);
        const f16 wg = (f16)(w * f16_bits_to_float(g[k]));
        if (wf) wf[n * H + k] = wg;
        ss += (double)(float)wg;
        cc += (double)w * (double)f16_bits_to_float(be[k]);
      }
      fs[n] = (float)ss;
      fc[n] = (float)(cc + (double)f16_bits_to_float(bias[n]));
    }
  }
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    const int b0 = kEmbParams + i * kPerLayer;
    const uint16_t* W = host.data() + L.off[b0 + 0];  // Q | K | V rows
    const uint16_t* bias = host.data() + L.off[b0 + 1];
    const f16* wf = nullptr;  // the folded copy, where gamma is not all ones
    const float *fs = nullptr, *fc = nullptr;
    for (size_t f = 0; f < folds.size(); ++f)
      if (folds[f].qkv && folds[f].layer == i) {
        fs = reinterpret_cast<const float*>(buf.data() + vec_at[f]);
        fc = fs + folds[f].n;
        if (!ones[f]) wf = reinterpret_cast<const f16*>(buf.data() + w_at[f]);
      }
    f16* wp = reinterpret_cast<f16*>(buf.data() + hm_at[i]);
    float* fsp = reinterpret_cast<float*>(buf.data() + align256(hm_at[i] + 3 * H * H * sizeof(f16)));
    float* fcp = fsp + 3 * H;
    for (size_t h = 0; h < (size_t)BBH_NUM_HEADS; ++h)
      for (size_t part = 0; part < 3; ++part)
        for (size_t d = 0; d < (size_t)BBH_HEAD_DIM; ++d) {
          const size_t dst = h * 3 * BBH_HEAD_DIM + part * BBH_HEAD_DIM + d;
          const size_t src = part * H + h * BBH_HEAD_DIM + d;
          if (wf)
            memcpy(wp + dst * H, wf + src * H, H * sizeof(f16));
          else
            memcpy(wp + dst * H, W + src * H, H * sizeof(f16));
          fsp[dst] = fs ? fs[src] : 0.f;
          fcp[dst] = fc ? fc[src] : f16_bits_to_float(bias[src]);
        }
  }
  void* dev = nullptr;
  BBH_HIP(hipMalloc(&dev, cur), "hipMalloc(carried LayerNorm operands)");
  const hipError_t e = hipMemcpy(dev, buf.data(), cur, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    return hip_fail(e, "hipMemcpy(carried LayerNorm operands)");
  }
  m->fold_blob = dev;
  m->fold_bytes = cur;
  const unsigned char* base = static_cast<const unsigned char*>(dev);
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    auto& l = m->layers[i];
    l.qkv_wp = reinterpret_cast<const f16*>(base + hm_at[i]);
    l.qkv_fsp = reinterpret_cast<const float*>(base + align256(hm_at[i] + 3 * H * H * sizeof(f16)));
    l.qkv_fcp = l.qkv_fsp + 3 * H;
  }
  for (size_t f = 0; f < folds.size(); ++f) {
    auto& l = m->layers[folds[f].layer];
    const float* fs = reinterpret_cast<const float*>(base + vec_at[f]);
    const f16* wf = ones[f] ? nullptr : reinterpret_cast<const f16*>(base + w_at[f]);
    if (folds[f].qkv) {
      l.qkv_fs = fs;
      l.qkv_fc = fs + folds[f].n;
      l.qkv_wf = wf ? wf : l.qkv_w;
    } else {
      l.f1_fs = fs;
      l.f1_fc = fs + folds[f].n;
      l.f1_wf = wf ? wf : l.f1_w;
    }
  }
  return BBH_OK;
}

bbh_status model_from_host_blob(const std::vector<uint16_t>& host, bbh_model** out) {
  const BlobLayout& L = layout();
  bbh_model* m = new bbh_model();
  m->bytes = L.total * sizeof(f16);
  hipError_t e = hipMalloc(&m->blob, m->bytes);
  if (e != hipSuccess) {
    delete m;
    return fail(BBH_ERR_OOM, std::string("hipMalloc(weights): ") + hipGetErrorString(e));
  }
  e = hipMemcpy(m->blob, host.data(), m->bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(m->blob);
    delete m;
    return hip_fail(e, "hipMemcpy(weights)");
  }
  const f16* base = static_cast<const f16*>(m->blob);
  auto at = [&](int idx) { return base + L.off[idx]; };
  m->word = at(0);
  m->pos = at(1);
  m->type = at(2);
  m->emb_g = at(3);
  m->emb_b = at(4);
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    const int b0 = kEmbParams + i * kPerLayer;
    auto& l = m->layers[i];
    l.qkv_w = at(b0 + 0);
    l.qkv_b = at(b0 + 1);
    l.o_w = at(b0 + 6);
    l.o_b = at(b0 + 7);
    l.ln1_g = at(b0 + 8);
    l.ln1_b = at(b0 + 9);
    l.f1_w = at(b0 + 10);
    l.f1_b = at(b0 + 11);
    l.f2_w = at(b0 + 12);
    l.f2_b = at(b0 + 13);
    l.ln2_g = at(b0 + 14);
    l.ln2_b = at(b0 + 15);
  }
  const bbh_status st = fold_operands(host, m);
  if (st != BBH_OK) {
    (void)hipFree(m->blob);
    delete m;
    return st;
  }
  *out = m;
  return BBH_OK;
}

hipStream_t S(bbh_stream_t s) { return static_cast<hipStream_t>(s); }

bbh_status check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return hip_fail(e, what);
  return BBH_OK;
}

#define BBH_TRY(expr)                    \
  do {                                   \
    bbh_status _s = (expr);              \
    if (_s != BBH_OK) return _s;         \
  } while (0)

bbh_status check_shape(const bbh_workspace* ws, int batch, int seq) {
  if (batch < 1 || seq < 1)
    return fail(BBH_ERR_INVALID_ARG,
                "batch and seq must be positive (batch=" + std::to_string(batch) +
                    ", seq=" + std::to_string(seq) + ")");
  if (seq % BBH_SEQ_ALIGN != 0)
    return fail(BBH_ERR_SEQ_ALIGN, "seq must be a multiple of 16 (seq=" + std::to_string(seq) + ")");
  if (seq > BBH_MAX_POSITION)
    return fail(BBH_ERR_CAPACITY, "seq " + std::to_string(seq) + " exceeds max position 512");
  if (ws) {
    if (seq > ws->max_seq)
      return fail(BBH_ERR_CAPACITY, "seq " + std::to_string(seq) + " exceeds workspace max_seq " +
                                        std::to_string(ws->max_seq));
    if ((size_t)batch * seq > ws->rows)
      return fail(BBH_ERR_CAPACITY,
                  "batch*seq " + std::to_string((size_t)batch * seq) +
                      " exceeds workspace capacity " + std::to_string(ws->rows) + " rows");
  }
  return BBH_OK;
}

bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

bbh_status misaligned(const char* what) {
  return fail(BBH_ERR_INVALID_ARG, std::string(what) + ": device pointer not aligned for vector access");
}

const float kScale = 0.17677669529663687f;  // 1 / sqrt(32), src/model/encoder.cu:28

// Pairs of timing events around op launches (bbh_pool_timing).
struct OpTimer {
  std::vector<hipEvent_t> ev;  // two per slot
  std::vector<bbh_launch_time> rec;
  int used = 0;
  ~OpTimer() {
    for (auto e : ev) (void)hipEventDestroy(e);
  }
};

// launch() between a pair of events on s when t has a free slot.
template <class F>
bbh_status timed_op(OpTimer* t, hipStream_t s, const bbh_launch_time& meta, F&& launch) {
  int slot = -1;
  if (t && t->used < (int)t->rec.size() && hipEventRecord(t->ev[2 * t->used], s) == hipSuccess)
    slot = t->used++;
  const bbh_status st = launch();
  if (slot >= 0) {
    t->rec[slot] = meta;
    (void)hipEventRecord(t->ev[2 * slot + 1], s);
  }
  return st;
}

// A run of sentences with one padded length inside a forward: its masks, its
// shape, and its first row in the workspace's hidden buffers.  One forward
// may hold several segments: every Linear works per token, so the GEMMs run
// once over all rows and only attention, the embedding's positions and the
// pooling look at segment boundaries.
struct Segment {
  const int32_t* mask;
  int batch, seq;
  size_t row;
};

// A packed forward: n sentences (their plan in ws->sents), the longest max_len.
struct Packed {
  int n, max_len;
};

// out = LN(A . W^T + bias + residual) over 384-wide rows: one kernel where
// the GEMM tile owns whole rows, else the residual GEMM and a LayerNorm pass
// over out, timed as two ops.  With ln_deferred given, that LayerNorm pass is
// left to the caller (out holds the rows before it) and *ln_deferred says so.
bbh_status linear_residual_ln(OpTimer* t, hipStream_t s, int op, const f16* A, const f16* W,
                              const f16* bias, const f16* residual, const f16* gamma,
                              const f16* beta, f16* out, int M, int K, const char* what,
                              bool shared, bool* ln_deferred = nullptr) {
  const int H = BBH_HIDDEN;
  bool fused;
  const int tile = bbh::gemm_residual_ln_tile(M, K, &fused, shared);
  if (fused)
    return timed_op(t, s, {op, tile, 1, M, H, K, 0.f}, [&] {
      return check_launch(bbh::gemm_residual_ln(A, W, bias, residual, gamma, beta, out, M, K,
                                                BBH_LAYER_NORM_EPS, s, shared),
                          what);
    });
  BBH_TRY(timed_op(t, s, {op, tile, 0, M, H, K, 0.f}, [&] {
    return check_launch(bbh::gemm_residual(A, W, bias, residual, out, M, K, s, shared), what);
  }));
  if (ln_deferred) {
    *ln_deferred = true;
    return BBH_OK;
  }
  return timed_op(t, s, {BBH_OP_LAYERNORM, -1, 0, M, H, 0, 0.f}, [&] {
    return check_launch(bbh::layernorm(out, nullptr, gamma, beta, out, M, H, BBH_LAYER_NORM_EPS, s),
                        "residual layernorm");
  });
}

// Attention of the forward's sentences from ws->qkv into ws->ctx: packed
// (pk) or per padded segment.
bbh_status run_attention(bbh_workspace* ws, const Segment* segs, int n_segs, hipStream_t s,
                         OpTimer* t, const Packed* pk) {
  const int H = BBH_HIDDEN;
  if (pk) {
    BBH_TRY(timed_op(t, s, {BBH_OP_ATTENTION, -1, 0, pk->n, pk->max_len, BBH_NUM_HEADS, 0.f}, [&] {
      return check_launch(bbh::attention_packed(ws->qkv, ws->sents, pk->n, ws->ctx, BBH_NUM_HEADS,
                                                pk->max_len, kScale, s),
                          "attention (packed)");
    }));
  }
  for (int g = 0; g < n_segs; ++g) {
    const Segment& sg = segs[g];
    BBH_TRY(timed_op(t, s, {BBH_OP_ATTENTION, -1, 0, sg.batch, sg.seq, BBH_NUM_HEADS, 0.f}, [&] {
      return check_launch(bbh::attention(ws->qkv + sg.row * 3 * H, sg.mask, ws->ctx + sg.row * H,
                                         sg.batch, BBH_NUM_HEADS, sg.seq, kScale, s),
                          "attention");
    }));
  }
  return BBH_OK;
}

bbh_status run_attention_block(bbh_workspace* ws, const bbh_model::Layer& L, const f16* hidden,
                               const Segment* segs, int n_segs, f16* out, int M, hipStream_t s,
                               OpTimer* t = nullptr, const Packed* pk = nullptr) {
  const int H = BBH_HIDDEN;
  BBH_TRY(timed_op(t, s, {BBH_OP_QKV, bbh::gemm_tile(M, 3 * H, H, ws->shared), 0, M, 3 * H, H,
                          0.f}, [&] {
    return check_launch(bbh::gemm(hidden, L.qkv_w, L.qkv_b, ws->qkv, M, 3 * H, H,
                                  bbh::Act::kNone, s, ws->shared),
                        "qkv gemm");
  }));
  BBH_TRY(run_attention(ws, segs, n_segs, s, t, pk));
  return linear_residual_ln(t, s, BBH_OP_O_PROJ_LN, ws->ctx, L.o_w, L.o_b, hidden, L.ln1_g,
                            L.ln1_b, out, M, H, "o-proj gemm+ln", ws->shared);
}

bbh_status run_attention_block(bbh_workspace* ws, const bbh_model::Layer& L, const f16* hidden,
                               const int32_t* mask, f16* out, int batch, int seq, hipStream_t s,
                               OpTimer* t = nullptr) {
  const Segment one{mask, batch, seq, 0};
  return run_attention_block(ws, L, hidden, &one, 1, out, batch * seq, s, t);
}

bbh_status run_ffn_rows(bbh_workspace* ws, const bbh_model::Layer& L, const f16* hidden,
                        f16* out, int M, hipStream_t s, OpTimer* t = nullptr,
                        bool* ln_deferred = nullptr) {
  const int H = BBH_HIDDEN, F = BBH_FFN_DIM;
  // One kernel for the block at large M; it moves rows in 16-byte pieces
  // (the GEMM path falls back to its any-alignment kernel instead).
  if (bbh::ffn_fused_ok(M) && aligned(hidden, 16) && aligned(out, 16))
    return timed_op(t, s, {BBH_OP_FFN, -1, 1, M, H, F, 0.f}, [&] {
      return check_launch(bbh::ffn_fused(hidden, L.f1_w, L.f1_b, L.f2_w, L.f2_b, L.ln2_g, L.ln2_b,
                                         out, M, BBH_LAYER_NORM_EPS, s),
                          "ffn (one kernel)");
    });
  BBH_TRY(timed_op(t, s, {BBH_OP_FFN1_GELU, bbh::gemm_tile(M, F, H, ws->shared), 0, M, F, H, 0.f},
                   [&] {
    return check_launch(bbh::gemm(hidden, L.f1_w, L.f1_b, ws->inter, M, F, H, bbh::Act::kGelu, s,
                                  ws->shared),
                        "ffn1 gemm");
  }));
  return linear_residual_ln(t, s, BBH_OP_FFN2_LN, ws->inter, L.f2_w, L.f2_b, hidden, L.ln2_g,
                            L.ln2_b, out, M, F, "ffn2 gemm+ln", ws->shared, ln_deferred);
}

bbh_status run_ffn_block(bbh_workspace* ws, const bbh_model::Layer& L, const f16* hidden,
                         f16* out, int batch, int seq, hipStream_t s, OpTimer* t = nullptr) {
  return run_ffn_rows(ws, L, hidden, out, batch * seq, s, t);
}

// The six layers over M rows with their LayerNorms carried as row
// statistics (bbh::LnCarry, M <= 8192): no LayerNorm pass between GEMMs.
// `h0` holds the embedding LayerNorm's output.  Layer i's O-proj writes its
// rows before ln1 to ws->attn_out (pairs in st_a); FFN1 normalises them on
// the fly (writing their mean / rstd to mr_a), and FFN2 adds them, through
// ln1, as its residual while writing the rows before ln2 (pairs in st_b),
// which layer i + 1's QKV and O-proj read the same way (mr_b).  The last
// layer writes final_out (which may be ws->attn_out: each residual chunk is
// read by the thread that then overwrites it); its ln2 follows as a pass over
// final_out, or is left to the caller (final_ln_deferred).  Timing records
// of the carried GEMMs have fused_ln 2, and of bbh::qkv_attention (one padded
// segment, seq <= 128) fused_ln 3 with (M, batch, seq).
bbh_status run_layers_carried(bbh_workspace* ws, const bbh_model* m, f16* h0, const Segment* segs,
                              int n_segs, const Packed* pk, int M, f16* final_out, hipStream_t s,
                              OpTimer* t, bool* final_ln_deferred) {
  const int H = BBH_HIDDEN, F = BBH_FFN_DIM;
  const float eps = BBH_LAYER_NORM_EPS;
  const bool sh = ws->shared;
  // One padded segment of at most 128 tokens a sentence: QKV and attention
  // as one kernel.
  const bool fused_qa = !pk && n_segs == 1 && segs[0].row == 0 &&
                        bbh::qkv_attention_ok(segs[0].batch, segs[0].seq) &&
                        aligned(segs[0].mask, 4);
  const f16* cur = h0;
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    const bbh_model::Layer& L = m->layers[i];
    const bbh_model::Layer* P = i > 0 ? &m->layers[i - 1] : nullptr;  // its ln2 normalises cur
    const bool last = i == BBH_NUM_LAYERS - 1;
    f16* nxt = last ? final_out : (cur == ws->ping ? ws->pong : ws->ping);
    const int qkv_tile = bbh::gemm_tile(M, 3 * H, H, sh);
    if (fused_qa) {
      // QKV Linear and attention in one kernel (timing record: fused_ln 3)
      bbh::LnCarry cy;
      if (P) {
        cy.st_in = ws->st_b;
        cy.mr_out = ws->mr_b;
      }
      BBH_TRY(timed_op(t, s, {BBH_OP_QKV, -1, 3, M, segs[0].batch, segs[0].seq, 0.f}, [&] {
        return check_launch(bbh::qkv_attention(cur, L.qkv_wp, L.qkv_fsp, L.qkv_fcp, cy,
                                               segs[0].mask, ws->ctx, segs[0].batch,
                                               segs[0].seq, kScale, eps, s),
                            "qkv + attention");
      }));
    } else if (!P) {
      BBH_TRY(timed_op(t, s, {BBH_OP_QKV, qkv_tile, 0, M, 3 * H, H, 0.f}, [&] {
        return check_launch(bbh::gemm(cur, L.qkv_w, L.qkv_b, ws->qkv, M, 3 * H, H,
                                      bbh::Act::kNone, s, sh),
                            "qkv gemm");
      }));
    } else {
      bbh::LnCarry cy;
      cy.st_in = ws->st_b;
      cy.mr_out = ws->mr_b;
      cy.fs = L.qkv_fs;
      cy.fc = L.qkv_fc;
      BBH_TRY(timed_op(t, s, {BBH_OP_QKV, qkv_tile, 2, M, 3 * H, H, 0.f}, [&] {
        return check_launch(bbh::gemm_fold(cur, L.qkv_wf, cy, ws->qkv, M, 3 * H, H,
                                           bbh::Act::kNone, eps, s, sh),
                            "qkv gemm (carried LayerNorm)");
      }));
    }
    if (!fused_qa) BBH_TRY(run_attention(ws, segs, n_segs, s, t, pk));
    bool fused;
    {
      bbh::LnCarry cy;
      cy.mr_in = P ? ws->mr_b : nullptr;
      cy.st_out = ws->st_a;
      BBH_TRY(timed_op(t, s, {BBH_OP_O_PROJ_LN, bbh::gemm_residual_ln_tile(M, H, &fused, sh), 2, M,
                              H, H, 0.f}, [&] {
        return check_launch(bbh::gemm_residual_stats(ws->ctx, L.o_w, L.o_b, cur,
                                                     P ? P->ln2_g : nullptr,
                                                     P ? P->ln2_b : nullptr, cy, ws->attn_out, M,
                                                     H, s, sh),
                            "o-proj gemm (row statistics)");
      }));
    }
    {
      bbh::LnCarry cy;
      cy.st_in = ws->st_a;
      cy.mr_out = ws->mr_a;
      cy.fs = L.f1_fs;
      cy.fc = L.f1_fc;
      BBH_TRY(timed_op(t, s, {BBH_OP_FFN1_GELU, bbh::gemm_tile(M, F, H, sh), 2, M, F, H, 0.f}, [&] {
        return check_launch(bbh::gemm_fold(ws->attn_out, L.f1_wf, cy, ws->inter, M, F, H,
                                           bbh::Act::kGelu, eps, s, sh),
                            "ffn1 gemm (carried LayerNorm)");
      }));
    }
    {
      bbh::LnCarry cy;
      cy.mr_in = ws->mr_a;
      cy.st_out = last ? nullptr : ws->st_b;
      BBH_TRY(timed_op(t, s, {BBH_OP_FFN2_LN, bbh::gemm_residual_ln_tile(M, F, &fused, sh), 2, M, H,
                              F, 0.f}, [&] {
        return check_launch(bbh::gemm_residual_stats(ws->inter, L.f2_w, L.f2_b, ws->attn_out,
                                                     L.ln1_g, L.ln1_b, cy, nxt, M, F, s, sh),
                            "ffn2 gemm (row statistics)");
      }));
    }
    cur = nxt;
  }
  if (final_ln_deferred) {
    *final_ln_deferred = true;
    return BBH_OK;
  }
  const bbh_model::Layer& L = m->layers[BBH_NUM_LAYERS - 1];
  return timed_op(t, s, {BBH_OP_LAYERNORM, -1, 0, M, H, 0, 0.f}, [&] {
    return check_launch(bbh::layernorm(final_out, nullptr, L.ln2_g, L.ln2_b, final_out, M, H, eps, s),
                        "residual layernorm");
  });
}

// Whether a forward of M rows carries its LayerNorms as row statistics.
bool carries_ln(const bbh_workspace* ws, int M) {
  return bbh::ln_carry_ok(M) && (size_t)M <= ws->carry_rows && ws->st_a;
}

// Embeddings + 6 layers over the segments' rows; the last layer writes
// `final_out` (which may be ws->attn_out: the FFN2+LN epilogue reads each
// residual element before the same thread overwrites it).  Segment g's
// tokens are at ids + tok[g] (types and masks likewise).  With
// final_ln_deferred given, a last LayerNorm that would run as a pass of its
// own is left to the caller (pool_out) and *final_ln_deferred says so.
bbh_status run_encode_segs(bbh_workspace* ws, const bbh_model* m, const int32_t* ids,
                           const int32_t* types, const int64_t* tok, const Segment* segs,
                           int n_segs, f16* final_out, hipStream_t s, OpTimer* t = nullptr,
                           bool* final_ln_deferred = nullptr) {
  if (final_ln_deferred) *final_ln_deferred = false;
  int M = 0;
  for (int g = 0; g < n_segs; ++g) {
    const Segment& sg = segs[g];
    BBH_TRY(timed_op(t, s, {BBH_OP_EMBED, -1, 0, sg.batch * sg.seq, sg.seq, 0, 0.f}, [&] {
      return check_launch(bbh::embedding_ln(ids + tok[g], types + tok[g], m->word, m->pos,
                                            m->type, m->emb_g, m->emb_b,
                                            ws->ping + sg.row * BBH_HIDDEN, sg.batch, sg.seq,
                                            BBH_LAYER_NORM_EPS, s),
                          "embedding+ln");
    }));
    M += sg.batch * sg.seq;
  }
  if (carries_ln(ws, M))
    return run_layers_carried(ws, m, ws->ping, segs, n_segs, nullptr, M, final_out, s, t,
                              final_ln_deferred);
  f16* cur = ws->ping;
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    f16* nxt = (i == BBH_NUM_LAYERS - 1) ? final_out : (cur == ws->ping ? ws->pong : ws->ping);
    BBH_TRY(run_attention_block(ws, m->layers[i], cur, segs, n_segs, ws->attn_out, M, s, t));
    BBH_TRY(run_ffn_rows(ws, m->layers[i], ws->attn_out, nxt, M, s, t,
                         i == BBH_NUM_LAYERS - 1 ? final_ln_deferred : nullptr));
    cur = nxt;
  }
  return BBH_OK;
}

// Embeddings + 6 layers over a packed forward of M rows (plan in ws->sents).
bbh_status run_encode_packed(bbh_workspace* ws, const bbh_model* m, const int32_t* ids,
                             const int32_t* types, const Packed& pk, int M, f16* final_out,
                             hipStream_t s, OpTimer* t = nullptr) {
  BBH_TRY(timed_op(t, s, {BBH_OP_EMBED, -1, 0, M, pk.max_len, 0, 0.f}, [&] {
    return check_launch(bbh::embedding_ln_packed(ids, types, m->word, m->pos, m->type, m->emb_g,
                                                 m->emb_b, ws->ping, ws->sents, pk.n,
                                                 BBH_LAYER_NORM_EPS, s),
                        "embedding+ln (packed)");
  }));
  if (M == 0) return BBH_OK;
  if (carries_ln(ws, M))
    return run_layers_carried(ws, m, ws->ping, nullptr, 0, &pk, M, final_out, s, t, nullptr);
  f16* cur = ws->ping;
  for (int i = 0; i < BBH_NUM_LAYERS; ++i) {
    f16* nxt = (i == BBH_NUM_LAYERS - 1) ? final_out : (cur == ws->ping ? ws->pong : ws->ping);
    BBH_TRY(run_attention_block(ws, m->layers[i], cur, nullptr, 0, ws->attn_out, M, s, t, &pk));
    BBH_TRY(run_ffn_rows(ws, m->layers[i], ws->attn_out, nxt, M, s, t));
    cur = nxt;
  }
  return BBH_OK;
}

bbh_status run_encode(bbh_workspace* ws, const bbh_model* m, const int32_t* ids,
                      const int32_t* types, const int32_t* mask, f16* final_out, int batch,
                      int seq, hipStream_t s, OpTimer* t = nullptr,
                      bool* final_ln_deferred = nullptr) {
  const Segment one{mask, batch, seq, 0};
  const int64_t tok0 = 0;
  return run_encode_segs(ws, m, ids, types, &tok0, &one, 1, final_out, s, t, final_ln_deferred);
}

// Masked mean pool + L2 normalise of a forward's final rows into out.  If the
// forward left its last LayerNorm to the pool (final_ln_deferred), the pool
// normalises each counted row itself, bit for bit as that pass would: one
// launch fewer.  For callers that do not hand out the hidden rows.
bbh_status pool_out(OpTimer* t, hipStream_t s, const bbh_model* m, bool ln_deferred,
                    const f16* hidden, const int32_t* mask, f16* out, int batch, int seq) {
  return timed_op(t, s, {BBH_OP_POOL, -1, 0, batch, seq, 0, 0.f}, [&] {
    const bbh_model::Layer& L = m->layers[BBH_NUM_LAYERS - 1];
    return check_launch(ln_deferred ? bbh::ln_pool_normalize(hidden, mask, L.ln2_g, L.ln2_b,
                                                             BBH_LAYER_NORM_EPS, out, batch, seq, s)
                                    : bbh::pool_normalize(hidden, mask, out, batch, seq, s),
                        "pool+normalize");
  });
}

}  // namespace

extern "C" {

const char* bbh_status_string(bbh_status s) {
  switch (s) {
    case BBH_OK: return "ok";
    case BBH_ERR_INVALID_ARG: return "invalid argument";
    case BBH_ERR_SEQ_ALIGN: return "seq not a multiple of 16";
    case BBH_ERR_CAPACITY: return "capacity exceeded";
    case BBH_ERR_IO: return "weight file error";
    case BBH_ERR_HIP: return "HIP runtime error";
    case BBH_ERR_OOM: return "device out of memory";
    case BBH_ERR_UNSUPPORTED: return "unsupported shape";
  }
  return "unknown status";
}

const char* bbh_last_error(void) { return g_err.c_str(); }

const char* bbh_version(void) { return "bbh 0.1 gfx950"; }

int bbh_param_count(void) { return (int)params().size(); }

const char* bbh_param_name(int index) {
  if (index < 0 || index >= (int)params().size()) return nullptr;
  return params()[index].name.c_str();
}

size_t bbh_param_numel(int index) {
  if (index < 0 || index >= (int)params().size()) return 0;
  return params()[index].numel;
}

bbh_status bbh_model_from_host(const uint16_t* const* tensors, int n_tensors, bbh_model** out) {
  if (!tensors || !out) return fail(BBH_ERR_INVALID_ARG, "null tensors/out");
  if (n_tensors != bbh_param_count())
    return fail(BBH_ERR_INVALID_ARG, "expected " + std::to_string(bbh_param_count()) +
                                         " tensors, got " + std::to_string(n_tensors));
  const auto& p = params();
  const BlobLayout& L = layout();
  std::vector<uint16_t> host(L.total, 0);
  for (int i = 0; i < n_tensors; ++i) {
    if (!tensors[i]) return fail(BBH_ERR_INVALID_ARG, "null tensor " + p[i].name);
    memcpy(host.data() + L.off[i], tensors[i], p[i].numel * sizeof(uint16_t));
  }
  return model_from_host_blob(host, out);
}

bbh_status bbh_model_load_dir(const char* dir, bbh_model** out) {
  if (!dir || !out) return fail(BBH_ERR_INVALID_ARG, "null dir/out");
  const auto& p = params();
  const BlobLayout& L = layout();
  std::vector<uint16_t> host(L.total, 0);
  for (size_t i = 0; i < p.size(); ++i) {
    const std::string path = std::string(dir) + "/" + p[i].name + ".bin";
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return fail(BBH_ERR_IO, "cannot open " + path);
    fseek(f, 0, SEEK_END);
    const long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    const size_t want = p[i].numel * sizeof(uint16_t);
    if (sz < 0 || (size_t)sz != want) {
      fclose(f);
      return fail(BBH_ERR_IO, path + ": expected " + std::to_string(want) + " bytes, found " +
                                  std::to_string(sz));
    }
    const size_t got = fread(host.data() + L.off[i], sizeof(uint16_t), p[i].numel, f);
    fclose(f);
    if (got != p[i].numel)
      return fail(BBH_ERR_IO, path + ": short read (" + std::to_string(got) + " of " +
                                  std::to_string(p[i].numel) + " elements)");
  }
  return model_from_host_blob(host, out);
}

// ---- safetensors ------------------------------------------------------------
// The container (huggingface/safetensors): an 8-byte little-endian header
// length N, N bytes of JSON mapping each tensor name to
// {"dtype", "shape", "data_offsets": [begin, end)} (offsets into the data
// section that follows the header), plus an optional "__metadata__" object.
namespace {

struct StTensor {
  std::string dtype;
  std::vector<int64_t> shape;
  int64_t begin = -1, end = -1;
};

// Just enough JSON for that header: objects, arrays, strings, integers and
// the literals; any other value is skipped structurally.
class Json {
 public:
  explicit Json(const std::string& s) : s_(s) {}
  bool ok() const { return ok_; }
  bool eat(char c) {
    ws();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  bool expect(char c) {
    if (!eat(c)) ok_ = false;
    return ok_;
  }
  std::string str() {
    std::string out;
    if (!expect('"')) return out;
    while (i_ < s_.size() && s_[i_] != '"') {
      char ch = s_[i_++];
      if (ch == '\\') {
        if (i_ >= s_.size()) break;
        const char e = s_[i_++];
        if (e == 'u') {  // \uXXXX: tensor names are ASCII; keep a placeholder
          i_ += 4;
          ch = '?';
        } else {
          ch = e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
        }
      }
      out += ch;
    }
    if (i_ > s_.size() || !eat('"')) ok_ = false;
    return out;
  }
  int64_t integer() {
    ws();
    size_t j = i_;
    const bool neg = j < s_.size() && s_[j] == '-';
    if (neg) ++j;
    int64_t v = 0;
    const size_t start = j;
    while (j < s_.size() && s_[j] >= '0' && s_[j] <= '9' && v < ((int64_t)1 << 56))
      v = v * 10 + (s_[j++] - '0');
    if (j == start) ok_ = false;
    i_ = j;
    return neg ? -v : v;
  }
  void skip(int depth = 0) {  // any value
    ws();
    if (!ok_ || i_ >= s_.size() || depth > 64) {
      ok_ = false;
      return;
    }
    const char c = s_[i_];
    if (c == '"') {
      str();
    } else if (c == '{' || c == '[') {
      const char close = c == '{' ? '}' : ']';
      ++i_;
      if (eat(close)) return;
      do {
        if (c == '{') {
          str();
          expect(':');
        }
        skip(depth + 1);
      } while (ok_ && eat(','));
      expect(close);
    } else {  // number or literal
      while (i_ < s_.size() && (isalnum((unsigned char)s_[i_]) || s_[i_] == '-' || s_[i_] == '+' ||
                                s_[i_] == '.'))
        ++i_;
    }
  }

 private:
  void ws() {
    while (i_ < s_.size() && isspace((unsigned char)s_[i_])) ++i_;
  }
  const std::string& s_;
  size_t i_ = 0;
  bool ok_ = true;
};

bool parse_st_header(const std::string& js, std::map<std::string, StTensor>& out) {
  Json j(js);
  if (!j.expect('{')) return false;
  if (j.eat('}')) return true;
  do {
    const std::string key = j.str();
    if (!j.expect(':')) return false;
    if (key == "__metadata__") {
      j.skip();
      continue;
    }
    StTensor t;
    if (!j.expect('{')) return false;
    if (!j.eat('}')) {
      do {
        const std::string k = j.str();
        if (!j.expect(':')) return false;
        if (k == "dtype") {
          t.dtype = j.str();
        } else if (k == "shape") {
          if (!j.expect('[')) return false;
          if (!j.eat(']')) {
            do t.shape.push_back(j.integer());
            while (j.ok() && j.eat(','));
            if (!j.expect(']')) return false;
          }
        } else if (k == "data_offsets") {
          if (!j.expect('[')) return false;
          t.begin = j.integer();
          if (!j.expect(',')) return false;
          t.end = j.integer();
          if (!j.expect(']')) return false;
        } else {
          j.skip();
        }
      } while (j.ok() && j.eat(','));
      if (!j.expect('}')) return false;
    }
    out[key] = t;
  } while (j.ok() && j.eat(','));
  return j.expect('}') && j.ok();
}

// IEEE binary16 bits of a float, round to nearest even (the host compiler's
// _Float16 conversion), and of a bfloat16 via its float value.
uint16_t f32_to_f16_bits(float v) {
  const _Float16 h = (_Float16)v;
  uint16_t b;
  memcpy(&b, &h, 2);
  return b;
}

}  // namespace

bbh_status bbh_model_load_safetensors(const char* path, bbh_model** out) {
  if (!path || !out) return fail(BBH_ERR_INVALID_ARG, "null path/out");
  FILE* f = fopen(path, "rb");
  if (!f) return fail(BBH_ERR_IO, std::string("cannot open ") + path);
  struct Closer {
    FILE* f;
    ~Closer() { fclose(f); }
  } closer{f};
  fseek(f, 0, SEEK_END);
  const long fsz = ftell(f);
  fseek(f, 0, SEEK_SET);
  unsigned char lenb[8];
  if (fsz < 8 || fread(lenb, 1, 8, f) != 8)
    return fail(BBH_ERR_IO, std::string(path) + ": not a safetensors file (no header length)");
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | lenb[i];
  if (hlen == 0 || hlen > (100u << 20) || 8 + hlen > (uint64_t)fsz)
    return fail(BBH_ERR_IO, std::string(path) + ": bad header length " + std::to_string(hlen));
  std::string header(hlen, '\0');
  if (fread(&header[0], 1, hlen, f) != hlen)
    return fail(BBH_ERR_IO, std::string(path) + ": short header");
  std::map<std::string, StTensor> tensors;
  if (!parse_st_header(header, tensors))
    return fail(BBH_ERR_IO, std::string(path) + ": malformed header JSON");
  const uint64_t data_size = (uint64_t)fsz - 8 - hlen;

  const auto& p = params();
  const BlobLayout& L = layout();
  std::vector<uint16_t> host(L.total, 0);
  std::vector<unsigned char> buf;
  for (size_t i = 0; i < p.size(); ++i) {
    auto it = tensors.find(p[i].name);
    if (it == tensors.end()) it = tensors.find("bert." + p[i].name);
    if (it == tensors.end())
      return fail(BBH_ERR_IO, std::string(path) + ": missing tensor " + p[i].name);
    const StTensor& t = it->second;
    const std::string where = std::string(path) + ": " + it->first;
    const size_t esz = t.dtype == "F32" ? 4 : (t.dtype == "F16" || t.dtype == "BF16") ? 2 : 0;
    if (esz == 0) return fail(BBH_ERR_IO, where + ": dtype " + t.dtype + " (want F32, F16 or BF16)");
    const std::vector<int64_t> want =
        p[i].rows ? std::vector<int64_t>{(int64_t)p[i].rows, (int64_t)(p[i].numel / p[i].rows)}
                  : std::vector<int64_t>{(int64_t)p[i].numel};
    if (t.shape != want) {
      std::string got;
      for (auto d : t.shape) got += (got.empty() ? "" : ",") + std::to_string(d);
      return fail(BBH_ERR_IO, where + ": shape [" + got + "]");
    }
    if (t.begin < 0 || t.end < t.begin || (uint64_t)t.end > data_size ||
        (uint64_t)(t.end - t.begin) != p[i].numel * esz)
      return fail(BBH_ERR_IO, where + ": data_offsets out of range or wrong size");
    buf.resize(p[i].numel * esz);
    if (fseek(f, (long)(8 + hlen + t.begin), SEEK_SET) != 0 ||
        fread(buf.data(), 1, buf.size(), f) != buf.size())
      return fail(BBH_ERR_IO, where + ": short read");
    uint16_t* dst = host.data() + L.off[i];
    if (t.dtype == "F16") {
      memcpy(dst, buf.data(), buf.size());
    } else if (t.dtype == "F32") {
      for (size_t e = 0; e < p[i].numel; ++e) {
        float v;
        memcpy(&v, buf.data() + 4 * e, 4);
        dst[e] = f32_to_f16_bits(v);
      }
    } else {  // BF16: the upper half of a float
      for (size_t e = 0; e < p[i].numel; ++e) {
        const uint32_t bits = (uint32_t)(buf[2 * e] | (buf[2 * e + 1] << 8)) << 16;
        float v;
        memcpy(&v, &bits, 4);
        dst[e] = f32_to_f16_bits(v);
      }
    }
  }
  return model_from_host_blob(host, out);
}

bbh_status bbh_model_free(bbh_model* m) {
  if (!m) return BBH_OK;
  hipError_t e = m->blob ? hipFree(m->blob) : hipSuccess;
  const hipError_t e2 = m->fold_blob ? hipFree(m->fold_blob) : hipSuccess;
  if (e == hipSuccess) e = e2;
  delete m;
  if (e != hipSuccess) return hip_fail(e, "hipFree(weights)");
  return BBH_OK;
}

size_t bbh_model_device_bytes(const bbh_model* m) { return m ? m->bytes + m->fold_bytes : 0; }

size_t bbh_workspace_bytes(int max_batch, int max_seq) {
  if (max_batch < 1 || max_seq < 1) return 0;
  const size_t rows = (size_t)max_batch * max_seq;
  const size_t H = BBH_HIDDEN;
  return align256(rows * 3 * H * 2) + align256(rows * BBH_FFN_DIM * 2) + 4 * align256(rows * H * 2) +
         align256(rows * sizeof(bbh::PackedSentence)) + carry_bytes(rows);
}

bbh_status bbh_workspace_create(int max_batch, int max_seq, bbh_workspace** out) {
  if (!out) return fail(BBH_ERR_INVALID_ARG, "null out");
  if (max_batch < 1 || max_seq < 1)
    return fail(BBH_ERR_INVALID_ARG, "max_batch and max_seq must be positive");
  if (max_seq % BBH_SEQ_ALIGN != 0)
    return fail(BBH_ERR_SEQ_ALIGN, "max_seq must be a multiple of 16");
  if (max_seq > BBH_MAX_POSITION)
    return fail(BBH_ERR_CAPACITY, "max_seq exceeds max position 512");
  if ((size_t)max_batch * max_seq > BBH_MAX_ROWS)
    return fail(BBH_ERR_CAPACITY, "max_batch*max_seq exceeds " + std::to_string(BBH_MAX_ROWS) +
                                      " rows");
  bbh_workspace* ws = new bbh_workspace();
  ws->max_batch = max_batch;
  ws->max_seq = max_seq;
  ws->rows = (size_t)max_batch * max_seq;
  ws->bytes = bbh_workspace_bytes(max_batch, max_seq);
  hipError_t e = hipMalloc(&ws->blob, ws->bytes);
  if (e != hipSuccess) {
    delete ws;
    return fail(BBH_ERR_OOM, std::string("hipMalloc(workspace): ") + hipGetErrorString(e));
  }
  char* p = static_cast<char*>(ws->blob);
  const size_t H = BBH_HIDDEN, rows = ws->rows;
  auto take = [&](size_t bytes) {
    f16* r = reinterpret_cast<f16*>(p);
    p += align256(bytes);
    return r;
  };
  ws->qkv = take(rows * 3 * H * 2);
  ws->inter = take(rows * BBH_FFN_DIM * 2);
  ws->ctx = take(rows * H * 2);
  ws->attn_out = take(rows * H * 2);
  ws->ping = take(rows * H * 2);
  ws->pong = take(rows * H * 2);
  ws->sents = reinterpret_cast<bbh::PackedSentence*>(take(rows * sizeof(bbh::PackedSentence)));
  ws->carry_rows = carry_rows(rows);
  ws->st_a = reinterpret_cast<float2*>(take(ws->carry_rows * bbh::kMaxCarryTiles * sizeof(float2)));
  ws->st_b = reinterpret_cast<float2*>(take(ws->carry_rows * bbh::kMaxCarryTiles * sizeof(float2)));
  ws->mr_a = reinterpret_cast<float2*>(take(ws->carry_rows * sizeof(float2)));
  ws->mr_b = reinterpret_cast<float2*>(take(ws->carry_rows * sizeof(float2)));
  *out = ws;
  return BBH_OK;
}

bbh_status bbh_workspace_free(bbh_workspace* ws) {
  if (!ws) return BBH_OK;
  hipError_t e = ws->blob ? hipFree(ws->blob) : hipSuccess;
  delete ws;
  if (e != hipSuccess) return hip_fail(e, "hipFree(workspace)");
  return BBH_OK;
}

void* bbh_workspace_hidden(bbh_workspace* ws) { return ws ? ws->attn_out : nullptr; }

bbh_status bbh_embed(bbh_workspace* ws, const bbh_model* m, const int32_t* ids,
                     const int32_t* types, const int32_t* mask, void* emb, int batch, int seq,
                     bbh_stream_t stream) {
  if (!ws || !m || !ids || !types || !mask || !emb)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embed: null argument");
  if (!aligned(emb, 4)) return misaligned("bbh_embed emb");
  BBH_TRY(check_shape(ws, batch, seq));
  const hipStream_t s = S(stream);
  BBH_TRY(run_encode(ws, m, ids, types, mask, ws->attn_out, batch, seq, s));
  return check_launch(bbh::pool_normalize(ws->attn_out, mask, static_cast<f16*>(emb), batch, seq, s),
                      "pool+normalize");
}

// ---- bbh_embed without a workspace ------------------------------------------
// The forward's activations in a file-scope device array instead of a
// workspace: BBH_NOALLOC_MAX_ROWS rows of the same six buffers (8,448 bytes a
// row) and the carried-LayerNorm statistics (112 bytes a row); 70.1 MB, which
// every GPU the library runs on holds until the process ends.  Host code never names the array in a kernel argument or copy: its
// address on each device comes from hipGetSymbolAddress, taken once per
// device with that device current (the entry point's first call there).
namespace {
constexpr size_t kScratchRowBytes =
    (3 * (size_t)BBH_HIDDEN + BBH_FFN_DIM + 4 * (size_t)BBH_HIDDEN) * sizeof(f16);
constexpr size_t kScratchBytes =
    (size_t)BBH_NOALLOC_MAX_ROWS * kScratchRowBytes + carry_bytes(BBH_NOALLOC_MAX_ROWS);
static_assert(BBH_NOALLOC_MAX_ROWS % 64 == 0, "each buffer stays 256-byte aligned");
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once taken

// The current device's copy of the scratch array (taken on first use).
bbh_status scratch_on_current_device(void** out) {
  int dev = -1;
  BBH_HIP(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(BBH_ERR_UNSUPPORTED, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    BBH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return fail(BBH_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BBH_OK;
}
}  // namespace

bbh_status bbh_embed_noalloc(const bbh_model* m, const int32_t* ids, const int32_t* types,
                             const int32_t* mask, void* emb, int batch, int seq,
                             bbh_stream_t stream) {
  if (!m || !ids || !types || !mask || !emb)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embed_noalloc: null argument");
  if (!aligned(emb, 4)) return misaligned("bbh_embed_noalloc emb");
  BBH_TRY(check_shape(nullptr, batch, seq));
  if ((size_t)batch * seq > BBH_NOALLOC_MAX_ROWS)
    return fail(BBH_ERR_CAPACITY, "bbh_embed_noalloc: batch*seq " +
                                      std::to_string((size_t)batch * seq) + " exceeds " +
                                      std::to_string(BBH_NOALLOC_MAX_ROWS) + " rows");
  void* base = nullptr;
  BBH_TRY(scratch_on_current_device(&base));
  // A workspace view of the array: the buffers bbh_workspace_create lays out,
  // sized for BBH_NOALLOC_MAX_ROWS rows.  Every buffer is written before it is
  // read within one forward, so nothing needs clearing between calls.
  bbh_workspace ws;
  ws.max_batch = BBH_NOALLOC_MAX_ROWS / BBH_SEQ_ALIGN;
  ws.max_seq = BBH_MAX_POSITION;
  ws.rows = BBH_NOALLOC_MAX_ROWS;
  ws.blob = nullptr;  // not owned
  ws.bytes = kScratchBytes;
  f16* p = static_cast<f16*>(base);
  const size_t R = BBH_NOALLOC_MAX_ROWS, H = BBH_HIDDEN;
  ws.qkv = p;
  ws.inter = ws.qkv + R * 3 * H;
  ws.ctx = ws.inter + R * BBH_FFN_DIM;
  ws.attn_out = ws.ctx + R * H;
  ws.ping = ws.attn_out + R * H;
  ws.pong = ws.ping + R * H;
  ws.sents = nullptr;  // padded forwards only
  ws.carry_rows = carry_rows(R);
  unsigned char* c = reinterpret_cast<unsigned char*>(ws.pong + R * H);
  auto take = [&](size_t bytes) {
    float2* r = reinterpret_cast<float2*>(c);
    c += align256(bytes);
    return r;
  };
  ws.st_a = take(ws.carry_rows * bbh::kMaxCarryTiles * sizeof(float2));
  ws.st_b = take(ws.carry_rows * bbh::kMaxCarryTiles * sizeof(float2));
  ws.mr_a = take(ws.carry_rows * sizeof(float2));
  ws.mr_b = take(ws.carry_rows * sizeof(float2));
  const hipStream_t s = S(stream);
  bool ln_deferred = false;  // no caller sees these rows
  BBH_TRY(run_encode(&ws, m, ids, types, mask, ws.attn_out, batch, seq, s, nullptr, &ln_deferred));
  return pool_out(nullptr, s, m, ln_deferred, ws.attn_out, mask, static_cast<f16*>(emb), batch,
                  seq);
}

struct bbh_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

static void graph_release(bbh_graph* g) {
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
}

bbh_status bbh_embed_graph_create(bbh_workspace* ws, const bbh_model* m, const int32_t* ids,
                                  const int32_t* types, const int32_t* mask, void* emb, int batch,
                                  int seq, bbh_graph** out) {
  if (!out) return fail(BBH_ERR_INVALID_ARG, "null out");
  *out = nullptr;
  if (!ws || !m || !ids || !types || !mask || !emb)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embed_graph_create: null argument");
  if (!aligned(emb, 4)) return misaligned("bbh_embed_graph_create emb");
  BBH_TRY(check_shape(ws, batch, seq));
  hipStream_t s = nullptr;
  BBH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  // One eager forward first: it validates the arguments and performs every
  // kernel's one-time launch set-up outside the capture.
  bbh_status st = bbh_embed(ws, m, ids, types, mask, emb, batch, seq, s);
  hipError_t e = hipSuccess;
  if (st == BBH_OK) e = hipStreamSynchronize(s);
  auto* g = new bbh_graph();
  if (st == BBH_OK && e == hipSuccess) e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (st == BBH_OK && e == hipSuccess) {
    st = bbh_embed(ws, m, ids, types, mask, emb, batch, seq, s);
    const hipError_t e2 = hipStreamEndCapture(s, &g->graph);  // ends the capture in every case
    if (st == BBH_OK) e = e2;
  }
  if (st == BBH_OK && e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  (void)hipStreamDestroy(s);
  if (st != BBH_OK || e != hipSuccess) {
    graph_release(g);
    return st != BBH_OK ? st : hip_fail(e, "graph capture");
  }
  *out = g;
  return BBH_OK;
}

bbh_status bbh_graph_launch(bbh_graph* g, bbh_stream_t stream) {
  if (!g || !g->exec) return fail(BBH_ERR_INVALID_ARG, "null graph");
  BBH_HIP(hipGraphLaunch(g->exec, S(stream)), "hipGraphLaunch");
  return BBH_OK;
}

bbh_status bbh_graph_free(bbh_graph* g) {
  if (g) graph_release(g);
  return BBH_OK;
}

bbh_status bbh_encode(bbh_workspace* ws, const bbh_model* m, const int32_t* ids,
                      const int32_t* types, const int32_t* mask, void* out, int batch, int seq,
                      bbh_stream_t stream) {
  if (!ws || !m || !ids || !types || !mask || !out)
    return fail(BBH_ERR_INVALID_ARG, "bbh_encode: null argument");
  BBH_TRY(check_shape(ws, batch, seq));
  return run_encode(ws, m, ids, types, mask, static_cast<f16*>(out), batch, seq, S(stream));
}

struct bbh_pool {
  int n_slots = 0;
  // Slots 0 .. n_slots-2 run on these streams; the last slot runs on the
  // stream of each call (slot_stream).
  std::vector<hipStream_t> streams;
  std::vector<hipEvent_t> done;  // per slot, recorded at the end of a call
  hipEvent_t fork = nullptr;
  std::vector<bbh_workspace*> ws;  // per slot
  // ws_free[j]: recorded by whichever stream last used workspace j, and
  // waited on by the next one, so calls made from different streams stay
  // ordered on the last slot's workspace.
  std::vector<hipEvent_t> ws_free;
  int device = 0;  // the device the pool was created on
  OpTimer* timer = nullptr;  // bbh_pool_timing
  int fail_at = -1;          // bbh_pool_fail_at (test hook)
  // bbh_embed_packed: plans go host -> device from pinned memory, two slots
  // used alternately by consecutive calls; a slot is rewritten only after the
  // copies that last read it (events per stream) have completed.
  struct Slot {
    bbh::PackedSentence* host = nullptr;
    size_t cap = 0;  // entries
    std::vector<hipEvent_t> copied;
    std::vector<bool> pending;
  } slot[2];
  int next_slot = 0;
  // Enqueue threads for slots 1 .. n-1 of bbh_embed_each, created with the
  // pool: each waits for a new generation, runs the job for its slot if the
  // call uses it, and reports back.
  struct Workers {
    std::vector<std::thread> th;
    std::mutex mu;
    std::condition_variable go, done;
    uint64_t gen = 0;
    int active = 0, remaining = 0;
    bool stop = false;
    std::function<void(int)> job;
  } wk;
};

namespace {

void worker_loop(bbh_pool* p, int j) {
  bbh_pool::Workers& w = p->wk;
  const bool dev_ok = hipSetDevice(p->device) == hipSuccess;
  uint64_t seen = 0;
  std::unique_lock<std::mutex> lk(w.mu);
  for (;;) {
    w.go.wait(lk, [&] { return w.stop || w.gen != seen; });
    if (w.stop) return;
    seen = w.gen;
    const bool mine = j < w.active;
    std::function<void(int)> f = w.job;
    lk.unlock();
    if (mine) {
      if (dev_ok)
        f(j);
      else
        f(-1 - j);  // reports that the thread could not make the device current
    }
    lk.lock();
    if (mine && --w.remaining == 0) w.done.notify_all();
  }
}

// Runs job(0) on the calling thread and job(j), 1 <= j < active, on the
// pool's threads; returns when all have finished.
void run_on_workers(bbh_pool* p, int active, const std::function<void(int)>& job) {
  bbh_pool::Workers& w = p->wk;
  {
    std::lock_guard<std::mutex> lk(w.mu);
    w.job = job;
    w.active = active;
    w.remaining = active - 1;
    ++w.gen;
  }
  w.go.notify_all();
  job(0);
  std::unique_lock<std::mutex> lk(w.mu);
  w.done.wait(lk, [&] { return w.remaining == 0; });
  w.job = nullptr;
}

// The fork/join of a pool call.  use(j, s) orders stream s after the last
// use of workspace j (and after the caller's prior work, for a pool stream);
// the destructor, on every exit of the call, records each used workspace's
// ws_free event on the stream that used it and makes the caller's stream
// wait for every pool stream the call forked: later work on the caller's
// stream (freeing emb, say) is ordered after everything the call enqueued,
// also when it fails part-way.  finish() does the same and reports errors.
// Slot j's stream in a pool call made on `caller`: the last slot runs on the
// caller's stream itself, the others on the pool's streams.  A one-slot pool
// thus runs on the caller's stream alone: on a stream of its own, joined into
// the caller's after every call, the same forwards ran ~0.7 us a kernel slower
// (varlen mix, 32 batches of 64 on one slot: 10.2 against 9.1 ms a pass; the
// same with event flags that drop the system-scope fence).  With n slots the
// caller's hardware queue runs a share instead of only waiting: HIP gives a
// process GPU_MAX_HW_QUEUES hardware queues (4 by default), so 4 slots keep
// every queue running a forward (varlen mix per batch: 5.07 -> 4.33 ms a
// pass against 3 pool streams beside an idle caller).
hipStream_t slot_stream(const bbh_pool* p, int j, hipStream_t caller) {
  return j == p->n_slots - 1 ? caller : p->streams[j];
}

class PoolCall {
 public:
  PoolCall(bbh_pool* p, hipStream_t caller) : p_(p), caller_(caller), stream_of_(p->ws.size()) {}
  ~PoolCall() { (void)finish(); }
  bbh_status begin() {
    BBH_HIP(hipEventRecord(p_->fork, caller_), "hipEventRecord(fork)");
    return BBH_OK;
  }
  bbh_status use(int j, hipStream_t s) {
    if (stream_of_[j]) return BBH_OK;
    if (s != caller_) BBH_HIP(hipStreamWaitEvent(s, p_->fork, 0), "hipStreamWaitEvent(fork)");
    BBH_HIP(hipStreamWaitEvent(s, p_->ws_free[j], 0), "hipStreamWaitEvent(workspace)");
    stream_of_[j] = s;
    return BBH_OK;
  }
  bbh_status finish() {
    bbh_status first = BBH_OK;
    auto keep = [&](hipError_t e, const char* what) {
      if (e != hipSuccess && first == BBH_OK) first = hip_fail(e, what);
    };
    for (size_t j = 0; j < stream_of_.size(); ++j) {
      const hipStream_t s = stream_of_[j];
      if (!s) continue;
      keep(hipEventRecord(p_->ws_free[j], s), "hipEventRecord(workspace)");
      if (s != caller_) {
        keep(hipEventRecord(p_->done[j], s), "hipEventRecord(join)");
        keep(hipStreamWaitEvent(caller_, p_->done[j], 0), "hipStreamWaitEvent(join)");
      }
      stream_of_[j] = nullptr;
    }
    return first;
  }

 private:
  bbh_pool* p_;
  hipStream_t caller_;
  std::vector<hipStream_t> stream_of_;  // per workspace: the stream that used it, or null
};

}  // namespace

static void pool_release(bbh_pool* p) {
  {
    std::lock_guard<std::mutex> lk(p->wk.mu);
    p->wk.stop = true;
  }
  p->wk.go.notify_all();
  for (auto& t : p->wk.th) t.join();
  for (auto st : p->streams) (void)hipStreamSynchronize(st);
  // the caller's stream may have used the last workspace
  for (auto e : p->ws_free) (void)hipEventSynchronize(e);
  for (auto& sl : p->slot) {
    for (auto e : sl.copied) (void)hipEventDestroy(e);
    if (sl.host) (void)hipHostFree(sl.host);
  }
  delete p->timer;
  for (auto w : p->ws) bbh_workspace_free(w);
  for (auto e : p->ws_free) (void)hipEventDestroy(e);
  for (auto e : p->done) (void)hipEventDestroy(e);
  for (auto s : p->streams) (void)hipStreamDestroy(s);
  if (p->fork) (void)hipEventDestroy(p->fork);
  delete p;
}

bbh_status bbh_pool_create(int n_streams, int max_batch, int max_seq, bbh_pool** out) {
  if (!out) return fail(BBH_ERR_INVALID_ARG, "null out");
  if (n_streams < 1 || n_streams > 64) return fail(BBH_ERR_INVALID_ARG, "n_streams must be in [1, 64]");
  bbh_pool* p = new bbh_pool();
  hipError_t e = hipGetDevice(&p->device);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&p->fork, hipEventDisableTiming);
  if (e != hipSuccess) {
    pool_release(p);
    return hip_fail(e, "hipEventCreate");
  }
  p->n_slots = n_streams;
  for (int i = 0; i < n_streams; ++i) {
    if (i < n_streams - 1) {  // the last slot runs on each call's own stream
      hipStream_t st;
      e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);  // default priority
      if (e != hipSuccess) {
        pool_release(p);
        return hip_fail(e, "hipStreamCreate");
      }
      p->streams.push_back(st);
    }
    for (auto* evs : {&p->done, &p->ws_free}) {
      hipEvent_t ev;
      e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (e != hipSuccess) {
        pool_release(p);
        return hip_fail(e, "hipEventCreate");
      }
      evs->push_back(ev);
    }
    bbh_workspace* w = nullptr;
    bbh_status st2 = bbh_workspace_create(max_batch, max_seq, &w);
    if (st2 != BBH_OK) {
      std::string msg = g_err;
      pool_release(p);
      return fail(st2, msg);
    }
    w->shared = n_streams > 1;
    p->ws.push_back(w);
    for (auto& sl : p->slot) {
      hipEvent_t ce;
      e = hipEventCreateWithFlags(&ce, hipEventDisableTiming);
      if (e != hipSuccess) {
        pool_release(p);
        return hip_fail(e, "hipEventCreate");
      }
      sl.copied.push_back(ce);
      sl.pending.push_back(false);
    }
  }
  try {
    for (int j = 1; j < n_streams; ++j) p->wk.th.emplace_back(worker_loop, p, j);
  } catch (const std::exception& ex) {
    pool_release(p);
    return fail(BBH_ERR_INVALID_ARG, std::string("pool threads: ") + ex.what());
  }
  *out = p;
  return BBH_OK;
}

bbh_status bbh_pool_fail_at(bbh_pool* pool, int batch) {
  if (!pool) return fail(BBH_ERR_INVALID_ARG, "null pool");
  pool->fail_at = batch < 0 ? -1 : batch;
  return BBH_OK;
}

bbh_status bbh_pool_busy(bbh_pool* pool, int* busy) {
  if (!pool || !busy) return fail(BBH_ERR_INVALID_ARG, "null argument");
  int n = 0;
  for (auto st : pool->streams) {
    const hipError_t e = hipStreamQuery(st);
    if (e == hipErrorNotReady)
      ++n;
    else if (e != hipSuccess)
      return hip_fail(e, "hipStreamQuery");
  }
  for (auto ev : pool->ws_free) {  // work a call ran on the caller's stream
    const hipError_t e = hipEventQuery(ev);
    if (e == hipErrorNotReady)
      ++n;
    else if (e != hipSuccess)
      return hip_fail(e, "hipEventQuery");
  }
  *busy = n;
  return BBH_OK;
}

bbh_status bbh_pool_free(bbh_pool* pool) {
  if (!pool) return BBH_OK;
  for (auto s : pool->streams) (void)hipStreamSynchronize(s);
  pool_release(pool);
  return BBH_OK;
}

bbh_status bbh_embed_batches(bbh_pool* pool, const bbh_model* m, const int32_t* ids,
                             const int32_t* types, const int32_t* mask,
                             const int64_t* tok_offsets, const int* batch_sizes, const int* seqs,
                             const int64_t* emb_rows, void* emb, int n_batches,
                             bbh_stream_t stream) {
  if (!pool || !m || !ids || !types || !mask || !tok_offsets || !batch_sizes || !seqs ||
      !emb_rows || !emb)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embed_batches: null argument");
  if (n_batches < 0) return fail(BBH_ERR_INVALID_ARG, "n_batches must be >= 0");
  const int n = pool->n_slots;
  // validate everything before enqueueing anything
  for (int i = 0; i < n_batches; ++i) {
    bbh_status st = check_shape(pool->ws[i % n], batch_sizes[i], seqs[i]);
    if (st != BBH_OK) return fail(st, "batch " + std::to_string(i) + ": " + g_err);
    if (tok_offsets[i] < 0 || emb_rows[i] < 0)
      return fail(BBH_ERR_INVALID_ARG, "batch " + std::to_string(i) + ": negative offset");
  }
  if (n_batches == 0) return BBH_OK;
  // Runs of consecutive batches with one seq that sit back to back in the
  // token arrays and in emb are one (sum of batches, seq) segment: sentences
  // are independent, so each keeps the embedding it gets alone while the
  // kernels see a larger M.  (Bit for bit where the LayerNorm path stays the
  // same; a larger M can move it into the GEMM epilogue, whose row
  // statistics sum in another order.)
  struct Run {
    int first, batch;
  };
  std::vector<Run> runs;
  // A run holds at most a workspace's rows.  (Splitting long runs to even out
  // the streams measured slower: smaller M costs more than the overlap gains.)
  const size_t cap = pool->ws[0]->rows;
  for (int i = 0; i < n_batches; ++i) {
    if (i > 0 && !runs.empty()) {
      Run& r = runs.back();
      const int k = i - 1;
      if (seqs[i] == seqs[k] &&
          tok_offsets[i] == tok_offsets[k] + (int64_t)batch_sizes[k] * seqs[k] &&
          emb_rows[i] == emb_rows[k] + batch_sizes[k] &&
          (size_t)(r.batch + batch_sizes[i]) * seqs[i] <= cap) {
        r.batch += batch_sizes[i];
        continue;
      }
    }
    runs.push_back({i, batch_sizes[i]});
  }
  // Runs are packed into groups, one forward each, up to a workspace's rows:
  // the GEMMs run over all rows of a group and only attention, the
  // embedding's positions and the pooling work per run.  Largest run first,
  // into a new group while there are fewer groups than streams, else into
  // the group with the fewest rows that still has room (a new one if none
  // has).  Groups then go largest first to the least-loaded stream.
  const int n_runs = (int)runs.size();
  auto rows_of = [&](int r) { return (size_t)runs[r].batch * seqs[runs[r].first]; };
  std::vector<int> by_size(n_runs);
  for (int r = 0; r < n_runs; ++r) by_size[r] = r;
  std::stable_sort(by_size.begin(), by_size.end(),
                   [&](int a, int b) { return rows_of(a) > rows_of(b); });
  struct Group {
    std::vector<int> runs;
    size_t rows = 0;
  };
  std::vector<Group> groups;
  for (int r : by_size) {
    int best = -1;
    if ((int)groups.size() >= n) {
      for (int g = 0; g < (int)groups.size(); ++g)
        if (groups[g].rows + rows_of(r) <= cap && (best < 0 || groups[g].rows < groups[best].rows))
          best = g;
    }
    if (best < 0) {
      groups.push_back({});
      best = (int)groups.size() - 1;
    }
    groups[best].runs.push_back(r);
    groups[best].rows += rows_of(r);
  }
  const int n_groups = (int)groups.size();
  std::vector<int> order(n_groups);
  for (int g = 0; g < n_groups; ++g) {
    order[g] = g;
    std::sort(groups[g].runs.begin(), groups[g].runs.end());  // batch order inside a group
  }
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return groups[a].rows > groups[b].rows; });
  std::vector<size_t> load(n, 0);
  std::vector<int> stream_of(n_groups);
  for (int g : order) {
    const int j = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    stream_of[g] = j;
    load[j] += groups[g].rows;
  }
  PoolCall call(pool, S(stream));
  BBH_TRY(call.begin());
  std::vector<Segment> segs;
  std::vector<int64_t> tok;
  for (int q = 0; q < n_groups; ++q) {
    const int g = order[q];
    if (q == pool->fail_at)
      return fail(BBH_ERR_INVALID_ARG, "bbh_pool_fail_at: group " + std::to_string(q));
    const int j = stream_of[g];
    const hipStream_t st = slot_stream(pool, j, S(stream));
    BBH_TRY(call.use(j, st));
    bbh_workspace* w = pool->ws[j];
    segs.clear();
    tok.clear();
    size_t row = 0;
    for (int r : groups[g].runs) {
      const int i = runs[r].first;
      segs.push_back({mask + tok_offsets[i], runs[r].batch, seqs[i], row});
      tok.push_back(tok_offsets[i]);
      row += rows_of(r);
    }
    bool ln_deferred = false;  // a pool's workspaces are its own
    BBH_TRY(run_encode_segs(w, m, ids, types, tok.data(), segs.data(), (int)segs.size(),
                            w->attn_out, st, pool->timer, &ln_deferred));
    for (size_t k = 0; k < segs.size(); ++k) {
      const int i = runs[groups[g].runs[k]].first;
      f16* out = static_cast<f16*>(emb) + emb_rows[i] * BBH_HIDDEN;
      BBH_TRY(pool_out(pool->timer, st, m, ln_deferred,
                       w->attn_out + segs[k].row * BBH_HIDDEN, segs[k].mask, out, segs[k].batch,
                       segs[k].seq));
    }
  }
  return call.finish();
}

bbh_status bbh_embed_each(bbh_pool* pool, const bbh_model* m, const int32_t* ids,
                          const int32_t* types, const int32_t* mask, const int64_t* tok_offsets,
                          const int* batch_sizes, const int* seqs, const int64_t* emb_rows,
                          void* emb, int n_batches, bbh_stream_t stream) {
  if (!pool || !m || !ids || !types || !mask || !tok_offsets || !batch_sizes || !seqs ||
      !emb_rows || !emb)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embed_each: null argument");
  if (n_batches < 0) return fail(BBH_ERR_INVALID_ARG, "n_batches must be >= 0");
  if (!aligned(emb, 4)) return misaligned("bbh_embed_each emb");
  const int n = pool->n_slots;
  for (int i = 0; i < n_batches; ++i) {
    bbh_status st = check_shape(pool->ws[0], batch_sizes[i], seqs[i]);
    if (st != BBH_OK) return fail(st, "batch " + std::to_string(i) + ": " + g_err);
    if (tok_offsets[i] < 0 || emb_rows[i] < 0)
      return fail(BBH_ERR_INVALID_ARG, "batch " + std::to_string(i) + ": negative offset");
  }
  if (n_batches == 0) return BBH_OK;
  // Batch i goes, in batch order, to the stream with the fewest rows so far.
  std::vector<size_t> load(n, 0);
  std::vector<int> stream_of(n_batches);
  for (int i = 0; i < n_batches; ++i) {
    const int j = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    stream_of[i] = j;
    load[j] += (size_t)batch_sizes[i] * seqs[i];
  }
  const hipStream_t caller = S(stream);
  PoolCall call(pool, caller);
  BBH_TRY(call.begin());
  const int used = n_batches < n ? n_batches : n;  // every batch so far went to an empty stream
  for (int j = 0; j < used; ++j) BBH_TRY(call.use(j, slot_stream(pool, j, caller)));
  auto one = [&](int i) -> bbh_status {
    if (i == pool->fail_at)
      return fail(BBH_ERR_INVALID_ARG, "bbh_pool_fail_at: batch " + std::to_string(i));
    const int j = stream_of[i];
    const hipStream_t st = slot_stream(pool, j, caller);
    bbh_workspace* w = pool->ws[j];
    const int32_t* mk = mask + tok_offsets[i];
    bool ln_deferred = false;  // a pool's workspaces are its own
    BBH_TRY(run_encode(w, m, ids + tok_offsets[i], types + tok_offsets[i], mk, w->attn_out,
                       batch_sizes[i], seqs[i], st, pool->timer, &ln_deferred));
    f16* out = static_cast<f16*>(emb) + emb_rows[i] * BBH_HIDDEN;
    return pool_out(pool->timer, st, m, ln_deferred, w->attn_out, mk, out, batch_sizes[i],
                    seqs[i]);
  };
  if (used > 1 && !pool->timer) {
    // Each stream's batches are enqueued by a host thread of its own: the
    // caller's thread takes stream 0, the pool's threads (created with the
    // pool) the others.  Enqueueing the ~44 launches of every batch from one
    // thread cost the host about as long as the GPU took to run them
    // (4.3-5.1 ms against 5.5 ms for the varlen mix on 3 streams); launches
    // on different streams do not serialise (1.9-2.0 ms).  With op timing
    // on, one thread enqueues everything, so the timer's records stay in
    // launch order.  A failing stream stops its own batches; the others run
    // theirs, and the join (on every exit) orders the caller's stream after
    // all of them.
    std::vector<bbh_status> res(used, BBH_OK);
    std::vector<std::string> err(used);
    run_on_workers(pool, used, [&](int j) {
      if (j < 0) {
        res[-1 - j] = BBH_ERR_HIP;
        err[-1 - j] = "hipSetDevice in a pool thread";
        return;
      }
      for (int i = 0; i < n_batches && res[j] == BBH_OK; ++i)
        if (stream_of[i] == j) res[j] = one(i);
      if (res[j] != BBH_OK) err[j] = g_err;
    });
    for (int j = 0; j < used; ++j)
      if (res[j] != BBH_OK) return fail(res[j], err[j]);
  } else {
    for (int i = 0; i < n_batches; ++i) BBH_TRY(one(i));
  }
  return call.finish();
}

bbh_status bbh_embed_packed(bbh_pool* pool, const bbh_model* m, const int32_t* ids,
                            const int32_t* types, const int64_t* tok_offsets,
                            const int* batch_sizes, const int* seqs, const int32_t* lengths,
                            const int64_t* emb_rows, void* emb, int n_batches,
                            bbh_stream_t stream) {
  if (!pool || !m || !ids || !types || !tok_offsets || !batch_sizes || !seqs || !lengths ||
      !emb_rows || !emb)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embed_packed: null argument");
  if (n_batches < 0) return fail(BBH_ERR_INVALID_ARG, "n_batches must be >= 0");
  if (!aligned(emb, 4)) return misaligned("bbh_embed_packed emb");
  const int n = pool->n_slots;
  const size_t cap = pool->ws[0]->rows;  // tokens and sentences per forward
  // The sentences in batch order, validated before anything is enqueued.
  std::vector<bbh::PackedSentence> all;
  size_t k = 0, total = 0;
  for (int i = 0; i < n_batches; ++i) {
    const std::string at = "batch " + std::to_string(i) + ": ";
    if (batch_sizes[i] < 0) return fail(BBH_ERR_INVALID_ARG, at + "negative batch size");
    if (seqs[i] < 1 || seqs[i] > BBH_MAX_POSITION)
      return fail(BBH_ERR_CAPACITY, at + "seq must be in [1, 512]");
    if (tok_offsets[i] < 0 || emb_rows[i] < 0)
      return fail(BBH_ERR_INVALID_ARG, at + "negative offset");
    for (int j = 0; j < batch_sizes[i]; ++j, ++k) {
      const int len = lengths[k];
      if (len < 0 || len > seqs[i])
        return fail(BBH_ERR_INVALID_ARG, at + "sentence " + std::to_string(j) + " length " +
                                             std::to_string(len) + " outside [0, seq]");
      // Every forward must fit a workspace; the split below starts a forward
      // at a sentence without looking at its length.
      if ((size_t)len > cap)
        return fail(BBH_ERR_CAPACITY, at + "sentence " + std::to_string(j) + " length " +
                                          std::to_string(len) + " exceeds the pool workspace's " +
                                          std::to_string(cap) + " rows");
      all.push_back({tok_offsets[i] + (int64_t)j * seqs[i], emb_rows[i] + j, 0, len});
      total += (size_t)len;
    }
  }
  const size_t n_sent = all.size();
  if (n_sent == 0) return BBH_OK;
  // Forwards: consecutive sentences, about total / n tokens each (one per
  // stream), none over a workspace's rows in tokens or in sentences.
  const size_t target = std::max<size_t>(1, (total + n - 1) / n);
  std::vector<size_t> cut{0};  // first sentence of each forward
  size_t toks = 0;
  for (size_t i = 0; i < n_sent; ++i) {
    const size_t len = (size_t)all[i].len;
    if (i > cut.back() && (toks + len > cap || i - cut.back() >= cap ||
                           (toks >= target && (int)cut.size() < n))) {
      cut.push_back(i);
      toks = 0;
    }
    toks += len;
  }
  cut.push_back(n_sent);
  const int n_fwd = (int)cut.size() - 1;
  // Plan rows and the pinned slot.
  bbh_pool::Slot& sl = pool->slot[pool->next_slot];
  pool->next_slot ^= 1;
  for (int j = 0; j < n; ++j)
    if (sl.pending[j]) {
      BBH_HIP(hipEventSynchronize(sl.copied[j]), "hipEventSynchronize(plan slot)");
      sl.pending[j] = false;
    }
  if (sl.cap < n_sent) {
    if (sl.host) BBH_HIP(hipHostFree(sl.host), "hipHostFree");
    sl.host = nullptr;
    sl.cap = 0;
    BBH_HIP(hipHostMalloc(reinterpret_cast<void**>(&sl.host), n_sent * sizeof(bbh::PackedSentence),
                          hipHostMallocDefault),
            "hipHostMalloc(plan)");
    sl.cap = n_sent;
  }
  for (int f = 0; f < n_fwd; ++f) {
    int32_t row = 0;
    for (size_t i = cut[f]; i < cut[f + 1]; ++i) {
      all[i].row = row;
      row += all[i].len;
    }
  }
  std::copy(all.begin(), all.end(), sl.host);
  PoolCall call(pool, S(stream));
  BBH_TRY(call.begin());
  for (int f = 0; f < n_fwd; ++f) {
    if (f == pool->fail_at)
      return fail(BBH_ERR_INVALID_ARG, "bbh_pool_fail_at: forward " + std::to_string(f));
    const int j = f % n;
    const hipStream_t st = slot_stream(pool, j, S(stream));
    BBH_TRY(call.use(j, st));
    bbh_workspace* w = pool->ws[j];
    const size_t first = cut[f], cnt = cut[f + 1] - cut[f];
    int M = 0, max_len = 0;
    for (size_t i = first; i < first + cnt; ++i) {
      M += all[i].len;
      max_len = std::max(max_len, all[i].len);
    }
    BBH_HIP(hipMemcpyAsync(w->sents, sl.host + first, cnt * sizeof(bbh::PackedSentence),
                           hipMemcpyHostToDevice, st),
            "hipMemcpyAsync(plan)");
    BBH_HIP(hipEventRecord(sl.copied[j], st), "hipEventRecord(plan copied)");
    sl.pending[j] = true;
    const Packed pk{(int)cnt, max_len};
    BBH_TRY(run_encode_packed(w, m, ids, types, pk, M, w->attn_out, st, pool->timer));
    BBH_TRY(timed_op(pool->timer, st, {BBH_OP_POOL, -1, 0, (int)cnt, max_len, 0, 0.f}, [&] {
      return check_launch(bbh::pool_normalize_packed(w->attn_out, w->sents, (int)cnt,
                                                     static_cast<f16*>(emb), st),
                          "pool+normalize (packed)");
    }));
  }
  return call.finish();
}

bbh_status bbh_pool_timing(bbh_pool* pool, int capacity) {
  if (!pool) return fail(BBH_ERR_INVALID_ARG, "null pool");
  if (capacity < 0 || capacity > (1 << 16))
    return fail(BBH_ERR_INVALID_ARG, "timing capacity must be in [0, 65536]");
  // the last slot's ops ran on a caller's stream: its workspace event follows them
  for (auto st : pool->streams) BBH_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
  for (auto e : pool->ws_free) BBH_HIP(hipEventSynchronize(e), "hipEventSynchronize");
  delete pool->timer;
  pool->timer = nullptr;
  if (capacity == 0) return BBH_OK;
  auto* t = new OpTimer;
  t->ev.assign(2 * (size_t)capacity, nullptr);
  for (auto& e : t->ev) {
    // Timestamps only: without the system-scope release fence an event record
    // is a marker, not a cache flush between the ops it brackets.
    const hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
    if (err != hipSuccess) {
      e = nullptr;
      delete t;
      return fail(BBH_ERR_HIP, std::string("hipEventCreate: ") + hipGetErrorName(err));
    }
  }
  t->rec.assign(capacity, bbh_launch_time{});
  pool->timer = t;
  return BBH_OK;
}

bbh_status bbh_pool_timing_read(bbh_pool* pool, bbh_launch_time* out, int max, int* count) {
  if (!pool || !count || (max > 0 && !out)) return fail(BBH_ERR_INVALID_ARG, "null argument");
  *count = 0;
  if (!pool->timer) return BBH_OK;
  for (auto st : pool->streams) BBH_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
  OpTimer* t = pool->timer;
  // The last slot runs on the caller's stream: wait for the events.
  for (int i = 0; i < t->used; ++i)
    BBH_HIP(hipEventSynchronize(t->ev[2 * i + 1]), "hipEventSynchronize");
  for (int i = 0; i < t->used; ++i)
    BBH_HIP(hipEventElapsedTime(&t->rec[i].ms, t->ev[2 * i], t->ev[2 * i + 1]),
            "hipEventElapsedTime");
  for (int i = 0; i < t->used && i < max; ++i) out[i] = t->rec[i];
  *count = t->used;
  return BBH_OK;
}

const char* bbh_gemm_tile_name(int tile) { return bbh::gemm_tile_name(tile); }

static bbh_status check_layer(const bbh_workspace* ws, const bbh_model* m, int layer,
                              const void* hidden, const void* out, int batch, int seq) {
  if (!ws || !m || !hidden || !out) return fail(BBH_ERR_INVALID_ARG, "null argument");
  if (layer < 0 || layer >= BBH_NUM_LAYERS)
    return fail(BBH_ERR_INVALID_ARG, "layer index " + std::to_string(layer) + " out of range");
  if (hidden == out) return fail(BBH_ERR_INVALID_ARG, "out may not alias hidden");
  if (!aligned(hidden, 16) || !aligned(out, 16)) return misaligned("hidden/out");
  return check_shape(ws, batch, seq);
}

// Caller-held weight views -> the internal per-layer pointer set (only the
// half a block reads is filled), with the alignment the kernels rely on.
static bbh_status layer_from(const bbh_attn_weights* a, const bbh_ffn_weights* f,
                             bbh_model::Layer* L) {
  *L = {};
  if (a) {
    if (!a->qkv_w || !a->qkv_b || !a->o_w || !a->o_b || !a->ln_w || !a->ln_b)
      return fail(BBH_ERR_INVALID_ARG, "null attention weight pointer");
    if (!aligned(a->qkv_w, 16) || !aligned(a->o_w, 16) || !aligned(a->qkv_b, 8) ||
        !aligned(a->o_b, 16) || !aligned(a->ln_w, 16) || !aligned(a->ln_b, 16))
      return misaligned("attention weights");
    L->qkv_w = static_cast<const f16*>(a->qkv_w);
    L->qkv_b = static_cast<const f16*>(a->qkv_b);
    L->o_w = static_cast<const f16*>(a->o_w);
    L->o_b = static_cast<const f16*>(a->o_b);
    L->ln1_g = static_cast<const f16*>(a->ln_w);
    L->ln1_b = static_cast<const f16*>(a->ln_b);
  }
  if (f) {
    if (!f->inter_w || !f->inter_b || !f->out_w || !f->out_b || !f->ln_w || !f->ln_b)
      return fail(BBH_ERR_INVALID_ARG, "null ffn weight pointer");
    if (!aligned(f->inter_w, 16) || !aligned(f->out_w, 16) || !aligned(f->inter_b, 8) ||
        !aligned(f->out_b, 16) || !aligned(f->ln_w, 16) || !aligned(f->ln_b, 16))
      return misaligned("ffn weights");
    L->f1_w = static_cast<const f16*>(f->inter_w);
    L->f1_b = static_cast<const f16*>(f->inter_b);
    L->f2_w = static_cast<const f16*>(f->out_w);
    L->f2_b = static_cast<const f16*>(f->out_b);
    L->ln2_g = static_cast<const f16*>(f->ln_w);
    L->ln2_b = static_cast<const f16*>(f->ln_b);
  }
  return BBH_OK;
}

static bbh_status check_block(const bbh_workspace* ws, const void* hidden, const void* out,
                              int batch, int seq) {
  if (!ws || !hidden || !out) return fail(BBH_ERR_INVALID_ARG, "null argument");
  if (hidden == out) return fail(BBH_ERR_INVALID_ARG, "out may not alias hidden");
  if (!aligned(hidden, 16) || !aligned(out, 16)) return misaligned("hidden/out");
  return check_shape(ws, batch, seq);
}

bbh_status bbh_model_layer(const bbh_model* m, int layer, bbh_attn_weights* attn,
                           bbh_ffn_weights* ffn) {
  if (!m) return fail(BBH_ERR_INVALID_ARG, "null model");
  if (layer < 0 || layer >= BBH_NUM_LAYERS)
    return fail(BBH_ERR_INVALID_ARG, "layer index " + std::to_string(layer) + " out of range");
  const bbh_model::Layer& L = m->layers[layer];
  if (attn) *attn = {L.qkv_w, L.qkv_b, L.o_w, L.o_b, L.ln1_g, L.ln1_b};
  if (ffn) *ffn = {L.f1_w, L.f1_b, L.f2_w, L.f2_b, L.ln2_g, L.ln2_b};
  return BBH_OK;
}

bbh_status bbh_attention_block_w(bbh_workspace* ws, const void* hidden, const bbh_attn_weights* w,
                                 const int32_t* mask, void* out, int batch, int seq,
                                 bbh_stream_t stream) {
  BBH_TRY(check_block(ws, hidden, out, batch, seq));
  if (!w || !mask) return fail(BBH_ERR_INVALID_ARG, "null weights or mask");
  bbh_model::Layer L;
  BBH_TRY(layer_from(w, nullptr, &L));
  return run_attention_block(ws, L, static_cast<const f16*>(hidden), mask, static_cast<f16*>(out),
                             batch, seq, S(stream));
}

bbh_status bbh_ffn_block_w(bbh_workspace* ws, const void* hidden, const bbh_ffn_weights* w,
                           void* out, int batch, int seq, bbh_stream_t stream) {
  BBH_TRY(check_block(ws, hidden, out, batch, seq));
  if (!w) return fail(BBH_ERR_INVALID_ARG, "null weights");
  bbh_model::Layer L;
  BBH_TRY(layer_from(nullptr, w, &L));
  return run_ffn_block(ws, L, static_cast<const f16*>(hidden), static_cast<f16*>(out), batch, seq,
                       S(stream));
}

bbh_status bbh_encoder_layer_w(bbh_workspace* ws, const void* hidden, const bbh_attn_weights* attn,
                               const bbh_ffn_weights* ffn, const int32_t* mask, void* out,
                               int batch, int seq, bbh_stream_t stream) {
  BBH_TRY(check_block(ws, hidden, out, batch, seq));
  if (!attn || !ffn || !mask) return fail(BBH_ERR_INVALID_ARG, "null weights or mask");
  if (out == ws->attn_out) return fail(BBH_ERR_INVALID_ARG, "out may not be the workspace's attn_out");
  bbh_model::Layer L;
  BBH_TRY(layer_from(attn, ffn, &L));
  const hipStream_t s = S(stream);
  BBH_TRY(run_attention_block(ws, L, static_cast<const f16*>(hidden), mask, ws->attn_out, batch,
                              seq, s));
  return run_ffn_block(ws, L, ws->attn_out, static_cast<f16*>(out), batch, seq, s);
}

bbh_status bbh_attention_block(bbh_workspace* ws, const bbh_model* m, int layer,
                               const void* hidden, const int32_t* mask, void* out, int batch,
                               int seq, bbh_stream_t stream) {
  BBH_TRY(check_layer(ws, m, layer, hidden, out, batch, seq));
  if (!mask) return fail(BBH_ERR_INVALID_ARG, "null mask");
  return run_attention_block(ws, m->layers[layer], static_cast<const f16*>(hidden), mask,
                             static_cast<f16*>(out), batch, seq, S(stream));
}

bbh_status bbh_ffn_block(bbh_workspace* ws, const bbh_model* m, int layer, const void* hidden,
                         void* out, int batch, int seq, bbh_stream_t stream) {
  BBH_TRY(check_layer(ws, m, layer, hidden, out, batch, seq));
  return run_ffn_block(ws, m->layers[layer], static_cast<const f16*>(hidden),
                       static_cast<f16*>(out), batch, seq, S(stream));
}

bbh_status bbh_encoder_layer(bbh_workspace* ws, const bbh_model* m, int layer,
                             const void* hidden, const int32_t* mask, void* out, int batch,
                             int seq, bbh_stream_t stream) {
  BBH_TRY(check_layer(ws, m, layer, hidden, out, batch, seq));
  if (!mask) return fail(BBH_ERR_INVALID_ARG, "null mask");
  if (out == ws->attn_out) return fail(BBH_ERR_INVALID_ARG, "out may not be the workspace's attn_out");
  const hipStream_t s = S(stream);
  BBH_TRY(run_attention_block(ws, m->layers[layer], static_cast<const f16*>(hidden), mask,
                              ws->attn_out, batch, seq, s));
  return run_ffn_block(ws, m->layers[layer], ws->attn_out, static_cast<f16*>(out), batch, seq, s);
}

bbh_status bbh_linear(const void* A, const void* B, void* C, int M, int N, int K,
                      const void* bias, int gelu, bbh_stream_t stream) {
  if (!A || !B || !C) return fail(BBH_ERR_INVALID_ARG, "bbh_linear: null operand");
  if (M < 1 || N < 1 || K < 1) return fail(BBH_ERR_INVALID_ARG, "bbh_linear: M, N, K must be positive");
  return check_launch(bbh::gemm(static_cast<const f16*>(A), static_cast<const f16*>(B),
                                static_cast<const f16*>(bias), static_cast<f16*>(C), M, N, K,
                                gelu ? bbh::Act::kGelu : bbh::Act::kNone, S(stream)),
                      "linear");
}

bbh_status bbh_linear_residual_layernorm(const void* A, const void* B, const void* bias,
                                         const void* residual, const void* gamma,
                                         const void* beta, void* y, int M, int N, int K,
                                         float eps, bbh_stream_t stream) {
  if (!A || !B || !bias || !residual || !gamma || !beta || !y)
    return fail(BBH_ERR_INVALID_ARG, "bbh_linear_residual_layernorm: null argument");
  if (M < 1 || K < 1) return fail(BBH_ERR_INVALID_ARG, "M and K must be positive");
  if (N != BBH_HIDDEN) return fail(BBH_ERR_UNSUPPORTED, "N must be 384");
  if (K % 64 != 0) return fail(BBH_ERR_UNSUPPORTED, "K must be a multiple of 64");
  if (!aligned(A, 16) || !aligned(B, 16) || !aligned(bias, 16) || !aligned(residual, 16) ||
      !aligned(gamma, 16) || !aligned(beta, 16) || !aligned(y, 16))
    return misaligned("bbh_linear_residual_layernorm");
  return check_launch(
      bbh::gemm_residual_ln(static_cast<const f16*>(A), static_cast<const f16*>(B),
                            static_cast<const f16*>(bias), static_cast<const f16*>(residual),
                            static_cast<const f16*>(gamma), static_cast<const f16*>(beta),
                            static_cast<f16*>(y), M, K, eps, S(stream)),
      "linear+residual+layernorm");
}

bbh_status bbh_layernorm(const void* x, const void* gamma, const void* beta, void* y, int M,
                         int D, float eps, const void* residual, bbh_stream_t stream) {
  if (!x || !gamma || !beta || !y) return fail(BBH_ERR_INVALID_ARG, "bbh_layernorm: null argument");
  if (M < 1 || D < 1 || D > 4096) return fail(BBH_ERR_INVALID_ARG, "bbh_layernorm: bad M/D");
  return check_launch(bbh::layernorm(static_cast<const f16*>(x), static_cast<const f16*>(residual),
                                     static_cast<const f16*>(gamma), static_cast<const f16*>(beta),
                                     static_cast<f16*>(y), M, D, eps, S(stream)),
                      "layernorm");
}

bbh_status bbh_embedding(const int32_t* ids, const int32_t* types, const void* word,
                         const void* pos, const void* type, void* out, int seq, int hidden,
                         int batch, bbh_stream_t stream) {
  if (!ids || !types || !word || !pos || !type || !out)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embedding: null argument");
  if (seq < 1 || hidden < 1 || batch < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  if (seq > BBH_MAX_POSITION) return fail(BBH_ERR_CAPACITY, "seq exceeds max position 512");
  return check_launch(bbh::embedding(ids, types, static_cast<const f16*>(word),
                                     static_cast<const f16*>(pos), static_cast<const f16*>(type),
                                     static_cast<f16*>(out), batch, seq, hidden, S(stream)),
                      "embedding");
}

bbh_status bbh_embedding_layernorm(const int32_t* ids, const int32_t* types, const void* word,
                                   const void* pos, const void* type, const void* gamma,
                                   const void* beta, void* out, int seq, int hidden, int batch,
                                   float eps, bbh_stream_t stream) {
  if (!ids || !types || !word || !pos || !type || !gamma || !beta || !out)
    return fail(BBH_ERR_INVALID_ARG, "bbh_embedding_layernorm: null argument");
  if (hidden != BBH_HIDDEN) return fail(BBH_ERR_UNSUPPORTED, "hidden must be 384");
  if (seq < 1 || batch < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  if (seq > BBH_MAX_POSITION) return fail(BBH_ERR_CAPACITY, "seq exceeds max position 512");
  if (!aligned(word, 4) || !aligned(pos, 4) || !aligned(type, 4) || !aligned(gamma, 4) ||
      !aligned(beta, 4) || !aligned(out, 4))
    return misaligned("bbh_embedding_layernorm");
  return check_launch(bbh::embedding_ln(ids, types, static_cast<const f16*>(word),
                                        static_cast<const f16*>(pos), static_cast<const f16*>(type),
                                        static_cast<const f16*>(gamma), static_cast<const f16*>(beta),
                                        static_cast<f16*>(out), batch, seq, eps, S(stream)),
                      "embedding+layernorm");
}

bbh_status bbh_attention(const void* qkv, const int32_t* mask, void* merged, int batch, int heads,
                         int seq, int head_dim, float scale, bbh_stream_t stream) {
  if (!qkv || !mask || !merged) return fail(BBH_ERR_INVALID_ARG, "bbh_attention: null argument");
  if (batch < 1 || heads < 1 || seq < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  if (head_dim != BBH_HEAD_DIM) return fail(BBH_ERR_UNSUPPORTED, "head_dim must be 32");
  if (seq % BBH_SEQ_ALIGN) return fail(BBH_ERR_SEQ_ALIGN, "seq must be a multiple of 16");
  if (seq > BBH_MAX_POSITION) return fail(BBH_ERR_CAPACITY, "seq exceeds 512");
  if (!aligned(qkv, 16) || !aligned(merged, 8)) return misaligned("bbh_attention");
  return check_launch(bbh::attention(static_cast<const f16*>(qkv), mask, static_cast<f16*>(merged),
                                     batch, heads, seq, scale, S(stream)),
                      "attention");
}

bbh_status bbh_attention_scores(const void* qkv, void* scores, int batch, int heads, int seq,
                                int head_dim, int qkv_stride, int q_off, int k_off, float scale,
                                bbh_stream_t stream) {
  if (!qkv || !scores) return fail(BBH_ERR_INVALID_ARG, "null argument");
  if (batch < 1 || heads < 1 || seq < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  if (head_dim != BBH_HEAD_DIM) return fail(BBH_ERR_UNSUPPORTED, "head_dim must be 32");
  if (seq % BBH_SEQ_ALIGN) return fail(BBH_ERR_SEQ_ALIGN, "seq must be a multiple of 16");
  if (qkv_stride % 8 || q_off % 8 || k_off % 8 || q_off < 0 || k_off < 0 ||
      q_off + heads * head_dim > qkv_stride || k_off + heads * head_dim > qkv_stride)
    return fail(BBH_ERR_INVALID_ARG, "qkv_stride/q_off/k_off must be multiples of 8 inside the row");
  if (!aligned(qkv, 16)) return misaligned("bbh_attention_scores");
  return check_launch(bbh::attention_scores(static_cast<const f16*>(qkv), static_cast<f16*>(scores),
                                            batch, heads, seq, qkv_stride, q_off, k_off, scale,
                                            S(stream)),
                      "attention_scores");
}

bbh_status bbh_softmax(void* x, int M, int N, const int32_t* mask, int mask_stride,
                       bbh_stream_t stream) {
  if (!x) return fail(BBH_ERR_INVALID_ARG, "null x");
  if (M < 1 || N < 1 || mask_stride < 0) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  return check_launch(bbh::softmax_rows(static_cast<f16*>(x), M, N, mask, mask_stride, S(stream)),
                      "softmax");
}

bbh_status bbh_attention_context(const void* probs, const void* qkv, void* merged, int batch,
                                 int heads, int seq, int head_dim, int qkv_stride, int v_off,
                                 bbh_stream_t stream) {
  if (!probs || !qkv || !merged) return fail(BBH_ERR_INVALID_ARG, "null argument");
  if (batch < 1 || heads < 1 || seq < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  if (head_dim != BBH_HEAD_DIM) return fail(BBH_ERR_UNSUPPORTED, "head_dim must be 32");
  if (v_off < 0 || v_off + heads * head_dim > qkv_stride)
    return fail(BBH_ERR_INVALID_ARG, "v_off outside the qkv row");
  return check_launch(bbh::attention_context(static_cast<const f16*>(probs),
                                             static_cast<const f16*>(qkv), static_cast<f16*>(merged),
                                             batch, heads, seq, qkv_stride, v_off, S(stream)),
                      "attention_context");
}

bbh_status bbh_mean_pool(const void* hidden, const int32_t* mask, void* out, int seq, int dim,
                         int batch, bbh_stream_t stream) {
  if (!hidden || !mask || !out) return fail(BBH_ERR_INVALID_ARG, "null argument");
  if (seq < 1 || dim < 1 || batch < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  return check_launch(bbh::mean_pool(static_cast<const f16*>(hidden), mask, static_cast<f16*>(out),
                                     batch, seq, dim, S(stream)),
                      "mean_pool");
}

bbh_status bbh_l2_normalize(void* x, int n, int batch, bbh_stream_t stream) {
  if (!x) return fail(BBH_ERR_INVALID_ARG, "null x");
  if (n < 1 || batch < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  return check_launch(bbh::l2_normalize(static_cast<f16*>(x), n, batch, S(stream)), "l2_normalize");
}

bbh_status bbh_pool_normalize(const void* hidden, const int32_t* mask, void* out, int seq, int dim,
                              int batch, bbh_stream_t stream) {
  if (!hidden || !mask || !out) return fail(BBH_ERR_INVALID_ARG, "null argument");
  if (dim != BBH_HIDDEN) return fail(BBH_ERR_UNSUPPORTED, "dim must be 384");
  if (seq < 1 || batch < 1) return fail(BBH_ERR_INVALID_ARG, "bad sizes");
  if (seq > BBH_MAX_POSITION) return fail(BBH_ERR_CAPACITY, "seq exceeds max position 512");
  if (!aligned(hidden, 4) || !aligned(out, 4)) return misaligned("bbh_pool_normalize");
  return check_launch(bbh::pool_normalize(static_cast<const f16*>(hidden), mask,
                                          static_cast<f16*>(out), batch, seq, S(stream)),
                      "pool+normalize");
}

bbh_status bbh_gelu(void* x, int n, bbh_stream_t stream) {
  if (n < 0) return fail(BBH_ERR_INVALID_ARG, "bbh_gelu: n must be >= 0");
  if (n == 0) return BBH_OK;
  if (!x) return fail(BBH_ERR_INVALID_ARG, "bbh_gelu: null x");
  return check_launch(bbh::gelu(static_cast<f16*>(x), (size_t)n, S(stream)), "gelu");
}

}  // extern "C"

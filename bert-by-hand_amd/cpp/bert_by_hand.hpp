// bert_by_hand.hpp - the reference's C++ host API, over the bbh C ABI.
//
// Same names, argument order, defaults and error behaviour as the headers of
// tytrdev/bert-by-hand:
//   src/core/model_config.h:5-22    model:: constants
//   src/core/cuda_check.h:7-24      abort-on-error checks (BBH_CHECK here)
//   src/core/device_buffer.h:7-63   DeviceBuffer
//   src/core/file_io.h:8-28         read_bin
//   src/core/loader.h:10-27         load_weight_fp16 / load_ref_i32 / load_ref_fp32
//   src/model/encoder.h:11-46       AttnWeights / FfnWeights / LayerWeights and the blocks
//   src/model/weights.h:15-107      ModelWeights, detail::load_qkv, load_model_weights
//   src/model/workspace.h:10-36     Workspace / make_workspace
//   src/model/forward.h:11-19       bert_encode / bert_embed
//   src/kernels/*.h                 launch_matmul, launch_layernorm, launch_softmax,
//                                   launch_attention_scores/_context, launch_embedding,
//                                   launch_mean_pool, launch_l2_normalize, launch_gelu
// Code written against those headers builds against this one with its
// include lines changed (and __half from <hip/hip_fp16.h>), links against
// libbbh.so and runs the gfx950 kernels.  As in the reference, every call
// enqueues on the null stream and returns without a host sync, and every
// error prints a message to stderr and aborts.
//
// Differences, all additive: make_workspace takes an optional max_seq
// (default SEQ_LEN = 128, the reference's fixed size) so seq up to 512 fits;
// every function takes an optional trailing hipStream_t; the Workspace's
// final hidden state is the view `attn_out` (data(), bytes()).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

#include "bbh.h"

namespace model {

constexpr int VOCAB_SIZE = BBH_VOCAB_SIZE;
constexpr int HIDDEN = BBH_HIDDEN;
constexpr int NUM_LAYERS = BBH_NUM_LAYERS;
constexpr int NUM_HEADS = BBH_NUM_HEADS;
constexpr int HEAD_DIM = BBH_HEAD_DIM;
constexpr int FFN_DIM = BBH_FFN_DIM;
constexpr int MAX_POSITION = BBH_MAX_POSITION;
constexpr int TYPE_VOCAB_SIZE = BBH_TYPE_VOCAB_SIZE;
constexpr float LAYER_NORM_EPS = BBH_LAYER_NORM_EPS;
constexpr int BATCH = 1;
constexpr int SEQ_LEN = 128;

constexpr const char *WEIGHTS_DIR = "weights";
constexpr const char *REF_DIR = "ref";

}  // namespace model

// A non-OK status of the C ABI: message to stderr, then abort().
#define BBH_CHECK(expr)                                                              \
  do {                                                                               \
    const bbh_status _st = (expr);                                                   \
    if (_st != BBH_OK) {                                                             \
      std::fprintf(stderr, "bbh error %s at %s:%d: %s\n", bbh_status_string(_st),    \
                   __FILE__, __LINE__, bbh_last_error());                            \
      std::abort();                                                                  \
    }                                                                                \
  } while (0)

// A failed HIP runtime call: message to stderr, then abort().
#define HIP_CHECK(expr)                                                              \
  do {                                                                               \
    const hipError_t _err = (expr);                                                  \
    if (_err != hipSuccess) {                                                        \
      std::fprintf(stderr, "HIP error %s at %s:%d: %s\n", hipGetErrorName(_err),     \
                   __FILE__, __LINE__, hipGetErrorString(_err));                     \
      std::abort();                                                                  \
    }                                                                                \
  } while (0)

// Only the launch status (no device sync): asynchronous faults surface at the
// next synchronising call, as with CUDA_CHECK_KERNEL.
#define HIP_CHECK_KERNEL() HIP_CHECK(hipGetLastError())

// ---- device memory (src/core/device_buffer.h) --------------------------------

// Move-only owner of one device allocation.
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t bytes) : bytes_(bytes) { HIP_CHECK(hipMalloc(&ptr_, bytes)); }
  ~DeviceBuffer() {
    if (ptr_) (void)hipFree(ptr_);
  }
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  DeviceBuffer(DeviceBuffer &&o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) {
    o.ptr_ = nullptr;
    o.bytes_ = 0;
  }
  DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
    if (this != &o) {
      if (ptr_) (void)hipFree(ptr_);
      ptr_ = o.ptr_;
      bytes_ = o.bytes_;
      o.ptr_ = nullptr;
      o.bytes_ = 0;
    }
    return *this;
  }

  void *data() { return ptr_; }
  const void *data() const { return ptr_; }
  size_t bytes() const { return bytes_; }

  // Blocking copies (they order after all work queued on the null stream).
  void from_host(const void *src, size_t n) {
    HIP_CHECK(hipMemcpy(ptr_, src, n, hipMemcpyHostToDevice));
  }
  void to_host(void *dst, size_t n) const {
    HIP_CHECK(hipMemcpy(dst, ptr_, n, hipMemcpyDeviceToHost));
  }

 private:
  void *ptr_ = nullptr;
  size_t bytes_ = 0;
};

// ---- files (src/core/file_io.h, src/core/loader.h) --------------------------

// Exactly expected_count raw little-endian values of T from path; a missing
// file, a short file or a longer file aborts with the path in the message.
template <typename T>
std::vector<T> read_bin(const std::string &path, size_t expected_count) {
  std::FILE *f = std::fopen(path.c_str(), "rb");
  if (!f) {
    std::fprintf(stderr, "read_bin: cannot open %s\n", path.c_str());
    std::abort();
  }
  std::vector<T> out(expected_count);
  const size_t got = std::fread(out.data(), sizeof(T), expected_count, f);
  const bool extra = std::fgetc(f) != EOF;
  std::fclose(f);
  if (got != expected_count || extra) {
    std::fprintf(stderr, "read_bin: %s: expected %zu elems, got %s%zu\n", path.c_str(),
                 expected_count, extra ? "more than " : "", got);
    std::abort();
  }
  return out;
}

inline DeviceBuffer load_weight_fp16(const std::string &name, size_t numel) {
  auto host = read_bin<uint16_t>(std::string(model::WEIGHTS_DIR) + "/" + name + ".bin", numel);
  DeviceBuffer buf(numel * sizeof(__half));
  buf.from_host(host.data(), host.size() * sizeof(uint16_t));
  return buf;
}

inline DeviceBuffer load_ref_i32(const std::string &name, size_t numel) {
  auto host = read_bin<int32_t>(std::string(model::REF_DIR) + "/" + name + ".bin", numel);
  DeviceBuffer buf(numel * sizeof(int32_t));
  buf.from_host(host.data(), host.size() * sizeof(int32_t));
  return buf;
}

inline std::vector<float> load_ref_fp32(const std::string &name, size_t numel) {
  return read_bin<float>(std::string(model::REF_DIR) + "/" + name + ".bin", numel);
}

// ---- weights (src/model/encoder.h:11-40, src/model/weights.h) ----------------

struct AttnWeights {
  const __half *qkv_w, *qkv_b;  // fused query/key/value projection
  const __half *o_w, *o_b;      // attention output dense
  const __half *ln_w, *ln_b;    // attention output LayerNorm
};

struct FfnWeights {
  const __half *inter_w, *inter_b;  // intermediate dense (HIDDEN -> FFN_DIM)
  const __half *out_w, *out_b;      // output dense (FFN_DIM -> HIDDEN)
  const __half *ln_w, *ln_b;        // output LayerNorm
};

struct LayerWeights {
  AttnWeights attn;
  FfnWeights ffn;
};

namespace detail {

inline bbh_attn_weights to_c(const AttnWeights &w) {
  return {w.qkv_w, w.qkv_b, w.o_w, w.o_b, w.ln_w, w.ln_b};
}
inline bbh_ffn_weights to_c(const FfnWeights &w) {
  return {w.inter_w, w.inter_b, w.out_w, w.out_b, w.ln_w, w.ln_b};
}

inline const __half *h(const DeviceBuffer &b) { return static_cast<const __half *>(b.data()); }

// Query, key and value tensors (`each` elements apiece) of layer prefix p,
// stacked along the output dimension in Q, K, V order.
inline DeviceBuffer load_qkv(const std::string &p, const char *suffix, size_t each) {
  static const char *parts[] = {"attention.self.query.", "attention.self.key.",
                                "attention.self.value."};
  std::vector<uint16_t> all(3 * each);
  for (int i = 0; i < 3; ++i) {
    auto v = read_bin<uint16_t>(std::string(model::WEIGHTS_DIR) + "/" + p + parts[i] + suffix +
                                    ".bin",
                                each);
    std::copy(v.begin(), v.end(), all.begin() + size_t(i) * each);
  }
  DeviceBuffer buf(all.size() * sizeof(uint16_t));
  buf.from_host(all.data(), all.size() * sizeof(uint16_t));
  return buf;
}

}  // namespace detail

// Every weight of the model in one device allocation owned by the library.
class ModelWeights {
 public:
  explicit ModelWeights(bbh_model *m = nullptr) : m_(m) {}
  ~ModelWeights() {
    if (m_) (void)bbh_model_free(m_);
  }
  ModelWeights(const ModelWeights &) = delete;
  ModelWeights &operator=(const ModelWeights &) = delete;
  ModelWeights(ModelWeights &&o) noexcept : m_(o.m_) { o.m_ = nullptr; }
  ModelWeights &operator=(ModelWeights &&o) noexcept {
    if (this != &o) {
      if (m_) (void)bbh_model_free(m_);
      m_ = o.m_;
      o.m_ = nullptr;
    }
    return *this;
  }

  // The pointer views of encoder layer i.
  LayerWeights layer(int i) const {
    bbh_attn_weights a;
    bbh_ffn_weights f;
    BBH_CHECK(bbh_model_layer(m_, i, &a, &f));
    auto hp = [](const void *p) { return static_cast<const __half *>(p); };
    return {{hp(a.qkv_w), hp(a.qkv_b), hp(a.o_w), hp(a.o_b), hp(a.ln_w), hp(a.ln_b)},
            {hp(f.inter_w), hp(f.inter_b), hp(f.out_w), hp(f.out_b), hp(f.ln_w), hp(f.ln_b)}};
  }

  const bbh_model *handle() const { return m_; }
  size_t device_bytes() const { return bbh_model_device_bytes(m_); }

 private:
  bbh_model *m_ = nullptr;
};

// <dir>/<state_dict name>.bin, raw fp16, 101 files (the pooler is not used).
inline ModelWeights load_model_weights(const std::string &dir = model::WEIGHTS_DIR) {
  bbh_model *m = nullptr;
  BBH_CHECK(bbh_model_load_dir(dir.c_str(), &m));
  return ModelWeights(m);
}

// ---- workspace (src/model/workspace.h) ---------------------------------------

// Scratch for forwards of up to (max_batch, max_seq), allocated once.  After
// bert_embed, attn_out holds the final hidden states (batch*seq, HIDDEN).
class Workspace {
 public:
  struct View {
    void *ptr = nullptr;
    size_t size = 0;
    void *data() const { return ptr; }
    size_t bytes() const { return size; }
  };

  explicit Workspace(bbh_workspace *ws = nullptr, size_t rows = 0) : ws_(ws) {
    if (ws_) attn_out = {bbh_workspace_hidden(ws_), rows * model::HIDDEN * sizeof(__half)};
  }
  ~Workspace() {
    if (ws_) (void)bbh_workspace_free(ws_);
  }
  Workspace(const Workspace &) = delete;
  Workspace &operator=(const Workspace &) = delete;
  Workspace(Workspace &&o) noexcept : attn_out(o.attn_out), ws_(o.ws_) {
    o.ws_ = nullptr;
    o.attn_out = {};
  }
  Workspace &operator=(Workspace &&o) noexcept {
    if (this != &o) {
      if (ws_) (void)bbh_workspace_free(ws_);
      ws_ = o.ws_;
      attn_out = o.attn_out;
      o.ws_ = nullptr;
      o.attn_out = {};
    }
    return *this;
  }

  bbh_workspace *handle() const { return ws_; }

  View attn_out;

 private:
  bbh_workspace *ws_ = nullptr;
};

inline Workspace make_workspace(int batch = 1, int max_seq = model::SEQ_LEN) {
  bbh_workspace *ws = nullptr;
  BBH_CHECK(bbh_workspace_create(batch, max_seq, &ws));
  return Workspace(ws, size_t(batch) * max_seq);
}

// ---- the forward (src/model/forward.h, src/model/encoder.h) ------------------

inline void bert_encode(Workspace &ws, const ModelWeights &w, const int32_t *input_ids,
                        const int32_t *token_type_ids, const int32_t *mask, __half *out,
                        int batch = 1, int seq = model::SEQ_LEN, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_encode(ws.handle(), w.handle(), input_ids, token_type_ids, mask, out, batch, seq,
                       stream));
}

inline void bert_embed(Workspace &ws, const ModelWeights &w, const int32_t *input_ids,
                       const int32_t *token_type_ids, const int32_t *mask, __half *embedding,
                       int batch = 1, int seq = model::SEQ_LEN, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_embed(ws.handle(), w.handle(), input_ids, token_type_ids, mask, embedding, batch,
                      seq, stream));
}

inline void attention_block(Workspace &ws, const __half *hidden, const AttnWeights &w,
                            const int32_t *mask, __half *out, int batch = 1,
                            int seq = model::SEQ_LEN, hipStream_t stream = nullptr) {
  const bbh_attn_weights c = detail::to_c(w);
  BBH_CHECK(bbh_attention_block_w(ws.handle(), hidden, &c, mask, out, batch, seq, stream));
}

inline void ffn_block(Workspace &ws, const __half *hidden, const FfnWeights &w, __half *out,
                      int batch = 1, int seq = model::SEQ_LEN, hipStream_t stream = nullptr) {
  const bbh_ffn_weights c = detail::to_c(w);
  BBH_CHECK(bbh_ffn_block_w(ws.handle(), hidden, &c, out, batch, seq, stream));
}

inline void encoder_layer(Workspace &ws, const __half *hidden, const LayerWeights &w,
                          const int32_t *mask, __half *out, int batch = 1,
                          int seq = model::SEQ_LEN, hipStream_t stream = nullptr) {
  const bbh_attn_weights a = detail::to_c(w.attn);
  const bbh_ffn_weights f = detail::to_c(w.ffn);
  BBH_CHECK(bbh_encoder_layer_w(ws.handle(), hidden, &a, &f, mask, out, batch, seq, stream));
}

// ---- kernel launchers (src/kernels/*.h) --------------------------------------

// C = A . B^T (+ bias) (then exact GELU); A (M,K), B (N,K) torch Linear layout.
inline void launch_matmul(const __half *A, const __half *B, __half *C, int M, int N, int K,
                          const __half *bias = nullptr, bool gelu = false,
                          hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_linear(A, B, C, M, N, K, bias, gelu ? 1 : 0, stream));
}

// Row LayerNorm of (x + residual) when residual != nullptr, else of x.
inline void launch_layernorm(const __half *x, const __half *gamma, const __half *beta, __half *y,
                             int M, int D, float eps, const __half *residual = nullptr,
                             hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_layernorm(x, gamma, beta, y, M, D, eps, residual, stream));
}

// Row softmax of (M, N) in place; mask columns with mask[j] == 0 are zeroed,
// mask_stride rows share one mask row (0: one mask for all rows).
inline void launch_softmax(__half *x, int M, int N, const int32_t *mask = nullptr,
                           int mask_stride = 0, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_softmax(x, M, N, mask, mask_stride, stream));
}

inline void launch_attention_scores(const __half *qkv, __half *scores, int batch, int heads,
                                    int seq, int head_dim, int qkv_stride, int q_off, int k_off,
                                    float scale, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_attention_scores(qkv, scores, batch, heads, seq, head_dim, qkv_stride, q_off,
                                 k_off, scale, stream));
}

inline void launch_attention_context(const __half *probs, const __half *qkv, __half *merged,
                                     int batch, int heads, int seq, int head_dim, int qkv_stride,
                                     int v_off, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_attention_context(probs, qkv, merged, batch, heads, seq, head_dim, qkv_stride,
                                  v_off, stream));
}

inline void launch_embedding(const int32_t *input_ids, const int32_t *token_type_ids,
                             const __half *word_emb, const __half *pos_emb,
                             const __half *type_emb, __half *out, int seq_len, int hidden,
                             int batch = 1, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_embedding(input_ids, token_type_ids, word_emb, pos_emb, type_emb, out, seq_len,
                          hidden, batch, stream));
}

inline void launch_mean_pool(const __half *hidden, const int32_t *mask, __half *out, int seq,
                             int dim, int batch = 1, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_mean_pool(hidden, mask, out, seq, dim, batch, stream));
}

inline void launch_l2_normalize(__half *x, int n, int batch = 1, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_l2_normalize(x, n, batch, stream));
}

inline void launch_gelu(__half *x, int n, hipStream_t stream = nullptr) {
  BBH_CHECK(bbh_gelu(x, n, stream));
}

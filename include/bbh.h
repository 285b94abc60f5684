/*
 * bbh.h - C ABI of the MI355X (gfx950) MiniLM-L6 sentence-embedding engine.
 *
 * This is the drop-in boundary for the reference's C++ host API
 * (tytrdev/bert-by-hand, src/model/ and src/kernels/ headers).  The reference
 * has no FFI layer of its own: its "operator API" is a set of C++ functions
 * taking __half / int32 device pointers.  Each entry point below names the
 * reference declaration it replaces.  A header-only C++ layer with the
 * reference's own names (ModelWeights, Workspace, load_model_weights,
 * make_workspace, bert_embed, ...) sits on top of this ABI in
 * bert-by-hand_amd/cpp/bert_by_hand.hpp.
 *
 * Conventions
 *  - All tensor arguments are DEVICE pointers.  fp16 data is IEEE binary16
 *    (passed as void* / uint16_t*), indices and masks are int32, row-major,
 *    and (batch, seq) inputs have row stride == seq.
 *  - Every call only enqueues work on `stream` (a hipStream_t; NULL = the
 *    null stream) and returns; the caller synchronises.  Nothing allocates
 *    device memory after bbh_model_* / bbh_workspace_create.
 *  - Every function returns a bbh_status.  On failure nothing is enqueued and
 *    bbh_last_error() returns a message for the calling thread.  (The
 *    reference instead prints and abort()s, src/core/cuda_check.h:7-17; the
 *    C++ layer restores that behaviour.)
 *  - A workspace must not be used by two calls that overlap in time.
 */
#ifndef BBH_H
#define BBH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model constants: src/core/model_config.h:7-17. */
#define BBH_VOCAB_SIZE 30522
#define BBH_HIDDEN 384
#define BBH_NUM_LAYERS 6
#define BBH_NUM_HEADS 12
#define BBH_HEAD_DIM 32
#define BBH_FFN_DIM 1536
#define BBH_MAX_POSITION 512
#define BBH_TYPE_VOCAB_SIZE 2
#define BBH_LAYER_NORM_EPS 1e-12f
#define BBH_SEQ_ALIGN 16   /* seq must be a multiple of this (bench/bench.cu:63) */
#define BBH_NUM_PARAMS 101 /* state_dict tensors without the pooler */
/* Most token rows (batch*seq) a workspace holds: 2048 x 512, which keeps
 * every rows x 1536 element count of the activations below 2^31. */
#define BBH_MAX_ROWS (1 << 20)

typedef enum bbh_status {
  BBH_OK = 0,
  BBH_ERR_INVALID_ARG = 1, /* null pointer, non-positive size, bad index */
  BBH_ERR_SEQ_ALIGN = 2,   /* seq % 16 != 0 */
  BBH_ERR_CAPACITY = 3,    /* batch / seq above the workspace or model limit */
  BBH_ERR_IO = 4,          /* weight file missing, unreadable or wrong size */
  BBH_ERR_HIP = 5,         /* HIP runtime error (message has the HIP name) */
  BBH_ERR_OOM = 6,         /* device allocation failed */
  BBH_ERR_UNSUPPORTED = 7  /* shape the kernels do not handle */
} bbh_status;

typedef struct bbh_model bbh_model;         /* device-resident weights */
typedef struct bbh_workspace bbh_workspace; /* device scratch for a forward */
typedef void *bbh_stream_t;                 /* hipStream_t */

/* ---- errors -------------------------------------------------------------- */
const char *bbh_status_string(bbh_status s);
/* Message of the last failed call on this thread ("" if none). */
const char *bbh_last_error(void);
const char *bbh_version(void);

/* ---- parameter table ------------------------------------------------------ */
/* The 101 tensors in HF state_dict order (scripts/dump_weights.py:75-83,
 * src/model/weights.h:56-107).  Names are the reference file stems. */
int bbh_param_count(void);
const char *bbh_param_name(int index);
size_t bbh_param_numel(int index);

/* ---- weights --------------------------------------------------------------
 * Replaces load_model_weights() (src/model/weights.h:88-107) with
 * load_weight_fp16 / read_bin (src/core/loader.h:10-16,
 * src/core/file_io.h:8-28): reads <dir>/<name>.bin raw little-endian fp16
 * files, checks each file size exactly, fuses Q|K|V along the output
 * dimension (src/model/weights.h:38-54) and uploads once.  Every file is read
 * and checked before any device memory is touched. */
bbh_status bbh_model_load_dir(const char *dir, bbh_model **out);
/* Same, from host fp16 arrays: tensors[i] points at bbh_param_numel(i)
 * binary16 values of tensor bbh_param_name(i). */
bbh_status bbh_model_from_host(const uint16_t *const *tensors, int n_tensors,
                               bbh_model **out);
/* The same model from a Hugging Face safetensors file (the model.safetensors
 * of a BertModel / sentence-transformers checkpoint; the reference exports the
 * same state dict to .bin files, scripts/dump_weights.py:69-94).  Tensors
 * named as above, optionally prefixed "bert."; dtype F32, F16 or BF16,
 * converted to fp16 with round-to-nearest-even; other tensors (the pooler)
 * are ignored.  Every tensor is found and checked (dtype, exact shape, byte
 * range) before any device memory is touched. */
bbh_status bbh_model_load_safetensors(const char *path, bbh_model **out);
bbh_status bbh_model_free(bbh_model *m);
size_t bbh_model_device_bytes(const bbh_model *m);

/* ---- workspace ------------------------------------------------------------
 * Replaces make_workspace(batch) (src/model/workspace.h:20-36).  The
 * reference sizes every buffer for SEQ_LEN = 128 tokens per row; here
 * max_seq is a runtime capacity (multiple of 16, at most 512) so batch 256 x
 * seq 512 fits; max_batch*max_seq <= BBH_MAX_ROWS.  All scratch for any
 * bbh_embed / bbh_encode with batch*seq <= max_batch*max_seq and
 * seq <= max_seq is allocated here, once. */
bbh_status bbh_workspace_create(int max_batch, int max_seq, bbh_workspace **out);
bbh_status bbh_workspace_free(bbh_workspace *ws);
size_t bbh_workspace_bytes(int max_batch, int max_seq);
/* Device pointer of the workspace's final-hidden buffer (batch*seq, 384)
 * fp16: after bbh_embed it holds the encoder output, as ws.attn_out does
 * after the reference's bert_embed (src/model/forward.cu:49). */
void *bbh_workspace_hidden(bbh_workspace *ws);

/* ---- the hot path ---------------------------------------------------------
 * bert_embed (src/model/forward.h:17-19, src/model/forward.cu:44-53):
 * embeddings -> 6 encoder layers -> masked mean pool -> L2 normalize.
 * ids/types/mask: (batch, seq) int32.  emb: (batch, 384) fp16.
 * seq is the runtime effective length, a multiple of 16, <= ws max_seq.
 * Token ids must lie in [0, 30522) and types in {0, 1}; out-of-range values
 * are clamped on the device rather than read out of bounds. */
bbh_status bbh_embed(bbh_workspace *ws, const bbh_model *m, const int32_t *ids,
                     const int32_t *types, const int32_t *mask, void *emb,
                     int batch, int seq, bbh_stream_t stream);
/* No counterpart in the reference: bbh_embed for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as bbh_embed
 * without the workspace: the forward's activations live in a device array of
 * the library (BBH_NOALLOC_MAX_ROWS rows, 70.1 MB on each GPU it runs on,
 * held until the process ends), so the call performs no allocation of any
 * kind on the success path.  batch*seq above BBH_NOALLOC_MAX_ROWS fails with
 * BBH_ERR_CAPACITY before anything is enqueued.  Every call on one GPU uses
 * the same array: calls that overlap in time on one GPU (two streams, two
 * threads) race and must be serialised by the caller.  The embeddings equal
 * bbh_embed's bit for bit. */
#define BBH_NOALLOC_MAX_ROWS 8192 /* batch 64 x seq 128 */
bbh_status bbh_embed_noalloc(const bbh_model *m, const int32_t *ids, const int32_t *types,
                             const int32_t *mask, void *emb, int batch, int seq,
                             bbh_stream_t stream);
/* bert_encode (src/model/forward.h:11-13, forward.cu:20-42): final hidden
 * states (batch*seq, 384) fp16 into out. */
bbh_status bbh_encode(bbh_workspace *ws, const bbh_model *m, const int32_t *ids,
                      const int32_t *types, const int32_t *mask, void *out,
                      int batch, int seq, bbh_stream_t stream);

/* ---- captured forwards ------------------------------------------------------
 * One forward is ~44 kernel launches.  bbh_embed_graph_create runs bbh_embed
 * once on a private stream, then
 * captures the same kernel sequence into a HIP graph; bbh_graph_launch
 * replays the whole forward as one launch on `stream`.  The graph is bound to
 * the buffers passed at creation (ids, types, mask, emb, the workspace and
 * the model): refill the inputs in place between launches.  Creation
 * synchronises its private stream; launches only enqueue.  Replays of one
 * graph, and any other call on its workspace, must not overlap in time.  This
 * saves the host its per-kernel launch calls (for callers that capture or
 * cannot afford them); on MI355X at batch 64 x seq 16 the GPU time per kernel
 * dominates, and replays measure no faster than eager bbh_embed. */
typedef struct bbh_graph bbh_graph;
bbh_status bbh_embed_graph_create(bbh_workspace *ws, const bbh_model *m, const int32_t *ids,
                                  const int32_t *types, const int32_t *mask, void *emb,
                                  int batch, int seq, bbh_graph **out);
bbh_status bbh_graph_launch(bbh_graph *g, bbh_stream_t stream);
bbh_status bbh_graph_free(bbh_graph *g);

/* ---- many batches ---------------------------------------------------------
 * A pool of n_streams slots, each with its own workspace of (max_batch,
 * max_seq).  The last slot runs on the stream a call is made on, the others
 * on n_streams - 1 HIP streams of the pool (default priority); a one-slot pool
 * thus runs on the caller's stream alone.  From 2 slots the GEMMs of a forward
 * use tiles chosen for a GPU shared with other forwards (the same results).
 * bbh_embed_batches runs bert_embed on n_batches batches spread over the
 * slots so that independent batches overlap on the GPU; it replaces the
 * reference's
 * sequential corpus loop (bench/corpus.cu:64-77,120-132).  Batch i reads its
 * (batch_sizes[i], seqs[i]) ids/types/mask starting at element
 * tok_offsets[i] of the device arrays and writes batch_sizes[i] rows of emb
 * starting at row emb_rows[i].  The size/offset arrays are HOST arrays.
 * Consecutive batches with the same seq that are adjacent both in the token
 * arrays and in emb form one run (one attention launch over their summed
 * batch), and runs are packed into groups of up to a pool workspace's
 * max_batch*max_seq rows: each group is one forward whose GEMMs cover all of
 * its rows, while attention, the embedding's positions and the pooling go
 * run by run.  A caller that packs equal-seq batches together thus gets
 * larger kernels with every batch's padding unchanged (the reference's corpus
 * benchmark instead re-sorts sentences by length, bench/corpus.cu:79-118).
 * Sentences never interact, so every sentence gets the embedding it gets
 * alone: bit for bit while its LayerNorm path is the one a lone batch takes,
 * else to within the rounding of the LayerNorm row statistics (larger groups
 * fuse the LayerNorm into the GEMM epilogue).  Groups are formed largest run
 * first, one per slot while slots remain, then into the group with the
 * fewest rows that has room; they go largest first to the least-loaded
 * slot.  The call orders itself after prior work on `stream` and makes
 * later work on `stream` wait for all batches; it returns without a host
 * sync.  On every return, errors included, everything the call enqueued is
 * ordered before later work on `stream`, so a caller may free emb or the
 * inputs on `stream` after a failed call.  Each pool workspace is also
 * ordered after its previous use, whichever stream made it, so calls on one
 * pool from different streams need no host sync between them; calls must
 * still not overlap in time on the host (a pool is not thread-safe).
 * bbh_pool_free waits for all of the pool's work, on any stream.  The pool
 * belongs to the device current at bbh_pool_create; with n_streams >= 2 it
 * also starts n_streams - 1 host threads (bbh_embed_each), stopped by
 * bbh_pool_free. */
typedef struct bbh_pool bbh_pool;
bbh_status bbh_pool_create(int n_streams, int max_batch, int max_seq, bbh_pool **out);
bbh_status bbh_pool_free(bbh_pool *pool);
/* Number of pool streams, plus workspaces last used on any stream, with
 * work still pending (0 when the pool is idle).  No counterpart in the
 * reference: for callers that poll instead of synchronising. */
bbh_status bbh_pool_busy(bbh_pool *pool, int *busy);
/* Test hook, no counterpart in the reference: later calls on this pool fail
 * with BBH_ERR_INVALID_ARG when they reach batch (bbh_embed_each), group
 * (bbh_embed_batches) or forward (bbh_embed_packed) number `batch`, after
 * enqueueing the earlier ones; a negative value switches it off.  For
 * exercising the error paths. */
bbh_status bbh_pool_fail_at(bbh_pool *pool, int batch);
bbh_status bbh_embed_batches(bbh_pool *pool, const bbh_model *m, const int32_t *ids,
                             const int32_t *types, const int32_t *mask,
                             const int64_t *tok_offsets, const int *batch_sizes,
                             const int *seqs, const int64_t *emb_rows, void *emb,
                             int n_batches, bbh_stream_t stream);

/* bbh_embed_each: the reference's corpus loop (bench/corpus.cu:64-77,
 * 120-132), one bert_embed per batch, with the batches spread over the pool
 * streams.  Same arguments as bbh_embed_batches, but every batch is its own
 * forward at its own (batch_sizes[i], seqs[i]) shape: nothing is merged and
 * every padding row is computed, so each batch's embeddings are bit for bit
 * those of bbh_embed on that batch.  Batch i goes, in batch order, to the
 * slot with the fewest rows so far.  Slots 0 .. n-2 run on the pool's
 * streams and slot n-1 on `stream` itself, so n = 4 keeps HIP's 4 hardware
 * queues per process (GPU_MAX_HW_QUEUES) busy.  The call orders itself after
 * prior work on `stream`, makes later work on `stream` wait for all batches,
 * and returns without a host sync.  With more than one slot in use (and op
 * timing off) each slot's launches are enqueued by a host thread of its own:
 * the caller's thread for slot 0, the pool's threads (created with the pool,
 * on the pool's device) for the others. */
bbh_status bbh_embed_each(bbh_pool *pool, const bbh_model *m, const int32_t *ids,
                          const int32_t *types, const int32_t *mask,
                          const int64_t *tok_offsets, const int *batch_sizes, const int *seqs,
                          const int64_t *emb_rows, void *emb, int n_batches,
                          bbh_stream_t stream);

/* bbh_embed_packed: the embeddings bbh_embed_batches gives for the same
 * batches when every mask is right padding (the tokenizer's layout: ones,
 * then zeros), computed without the padding rows.  lengths (HOST array, one
 * per sentence, batches in order) is each sentence's number of valid tokens,
 * in [0, seqs[i]]; the mask is not read.  Only valid tokens enter the
 * forward: the Linears and LayerNorms run over the sum of the lengths instead
 * of sum(batch_sizes[i] * seqs[i]) rows, and attention runs per sentence over
 * its own length (the reference pads every sentence of a batch to seq,
 * src/model/forward.cu:20-43).  Padding rows never reach a pooled embedding
 * (masked keys get zero weight, masked queries are left out of the mean), so
 * each embedding is the one bbh_embed_batches computes: bit for bit while
 * both forwards take the same LayerNorm path (a forward of more than 8192
 * rows fuses it into the GEMM epilogue), else to within the rounding of the
 * LayerNorm row statistics.  A sentence of length 0 gets a zero embedding.
 * Sentences are split, in order, into one forward per slot of about
 * equal token counts (more if a forward would exceed a workspace's
 * max_batch*max_seq tokens or sentences); seqs need not be multiples of 16.
 * A sentence longer than a workspace's max_batch*max_seq rows is rejected
 * with BBH_ERR_CAPACITY before anything is enqueued.
 * Each call uploads its sentence table from pinned memory; the call orders
 * itself after prior work on `stream`, makes later work on `stream` wait,
 * and returns without a host sync, except that it waits for the plan copies
 * of the call before last on this pool. */
bbh_status bbh_embed_packed(bbh_pool *pool, const bbh_model *m, const int32_t *ids,
                            const int32_t *types, const int64_t *tok_offsets,
                            const int *batch_sizes, const int *seqs, const int32_t *lengths,
                            const int64_t *emb_rows, void *emb, int n_batches,
                            bbh_stream_t stream);

/* ---- per-launch timing of a pool ---------------------------------------------
 * HIP-event timing of each op that bbh_embed_batches, bbh_embed_each and
 * bbh_embed_packed launch (the
 * reference times whole forwards with CUDA events, src/core/timer.h:36-39).
 * bbh_pool_timing(pool, capacity) starts a new record: a pair of events goes
 * on the launching stream around every op of every forward, for the
 * first `capacity` ops (later ones run untimed).  capacity 0 stops timing and
 * releases the events.  bbh_pool_timing_read waits for the recorded events, then
 * copies up to `max` records in launch order and sets *count to the number
 * recorded. */
typedef enum bbh_op {
  BBH_OP_QKV = 1,       /* fused QKV Linear */
  BBH_OP_ATTENTION = 2, /* masked multi-head attention */
  BBH_OP_O_PROJ_LN = 3, /* attention output Linear + residual (+ LayerNorm when fused) */
  BBH_OP_FFN1_GELU = 4, /* intermediate Linear + GELU */
  BBH_OP_FFN2_LN = 5,   /* output Linear + residual (+ LayerNorm when fused) */
  BBH_OP_EMBED = 6,     /* embedding gather + embedding LayerNorm */
  BBH_OP_POOL = 7,      /* masked mean pool + L2 normalize */
  BBH_OP_LAYERNORM = 8, /* residual LayerNorm pass after an unfused O-proj / FFN2, or the last
                           layer's when the LayerNorms are carried */
  BBH_OP_FFN = 9        /* the whole FFN block (intermediate Linear + GELU, output Linear +
                           residual + LayerNorm) in one kernel, at large M */
} bbh_op;
typedef struct bbh_launch_time {
  int op;       /* bbh_op */
  int tile;     /* GEMM tile configuration (bbh_gemm_tile_name); -1 for other ops */
  int fused_ln; /* 3 (BBH_OP_QKV only): the QKV Linear and the attention in one kernel (padded
                   forwards of at most 8192 rows and 128 tokens a sentence); no
                   BBH_OP_ATTENTION record follows, and m, n, k are (rows, batch, seq).
                   2: the LayerNorm carried as row statistics (forwards of at most 8192 rows):
                   O-proj / FFN2 write the rows before it with their statistics and no pass
                   follows; QKV (from layer 1) / FFN1 normalise their input rows from them.
                   O-proj / FFN2: 1 when the LayerNorm runs inside the GEMM kernel, 0 when it
                   follows as its own BBH_OP_LAYERNORM record */
  int m, n, k;  /* GEMM (M, N, K); attention (batch, seq, heads); embed / pool / LayerNorm
                   (rows or sentences, seq or 384, 0); FFN (M, 384, 1536) */
  float ms;     /* time between the pair of events */
} bbh_launch_time;
bbh_status bbh_pool_timing(bbh_pool *pool, int capacity);
bbh_status bbh_pool_timing_read(bbh_pool *pool, bbh_launch_time *out, int max, int *count);
/* "Cfg<BM,BN,WM,WN,SA,PD>" of a GEMM tile configuration, the template
 * argument in the kernel symbol gemm_kernel<Cfg<...>, epilogue>. */
const char *bbh_gemm_tile_name(int tile);

/* ---- weight views (src/model/encoder.h:11-22,37-40) -------------------------
 * Device pointers of one encoder layer's fp16 tensors, the reference's
 * AttnWeights / FfnWeights field for field.  Matrices, the output-dense
 * biases and the LayerNorm vectors must be 16-byte aligned (the fused
 * LayerNorm epilogues read them 16 bytes at a time), the QKV and intermediate
 * biases 8-byte aligned; every hipMalloc'd buffer is. */
typedef struct bbh_attn_weights {
  const void *qkv_w, *qkv_b; /* (1152, 384) with Q|K|V row blocks, (1152) */
  const void *o_w, *o_b;     /* attention output dense (384, 384), (384) */
  const void *ln_w, *ln_b;   /* attention output LayerNorm (384), (384) */
} bbh_attn_weights;
typedef struct bbh_ffn_weights {
  const void *inter_w, *inter_b; /* intermediate dense (1536, 384), (1536) */
  const void *out_w, *out_b;     /* output dense (384, 1536), (384) */
  const void *ln_w, *ln_b;       /* output LayerNorm (384), (384) */
} bbh_ffn_weights;
/* ModelWeights::layer(i) (src/model/weights.h:77-86): the views of encoder
 * layer `layer` of a loaded model.  Either output may be NULL. */
bbh_status bbh_model_layer(const bbh_model *m, int layer, bbh_attn_weights *attn,
                           bbh_ffn_weights *ffn);

/* ---- block level (src/model/encoder.h:27-46) ------------------------------
 * hidden / out: (batch*seq, 384) fp16, 16-byte aligned; mask (batch, seq)
 * int32.  out may not alias hidden.  The _w forms take the reference's
 * weight views; the others select layer `layer` of a loaded model. */
bbh_status bbh_attention_block_w(bbh_workspace *ws, const void *hidden,
                                 const bbh_attn_weights *w, const int32_t *mask,
                                 void *out, int batch, int seq, bbh_stream_t stream);
bbh_status bbh_ffn_block_w(bbh_workspace *ws, const void *hidden,
                           const bbh_ffn_weights *w, void *out, int batch, int seq,
                           bbh_stream_t stream);
bbh_status bbh_encoder_layer_w(bbh_workspace *ws, const void *hidden,
                               const bbh_attn_weights *attn, const bbh_ffn_weights *ffn,
                               const int32_t *mask, void *out, int batch, int seq,
                               bbh_stream_t stream);
bbh_status bbh_attention_block(bbh_workspace *ws, const bbh_model *m, int layer,
                               const void *hidden, const int32_t *mask, void *out,
                               int batch, int seq, bbh_stream_t stream);
bbh_status bbh_ffn_block(bbh_workspace *ws, const bbh_model *m, int layer,
                         const void *hidden, void *out, int batch, int seq,
                         bbh_stream_t stream);
bbh_status bbh_encoder_layer(bbh_workspace *ws, const bbh_model *m, int layer,
                             const void *hidden, const int32_t *mask, void *out,
                             int batch, int seq, bbh_stream_t stream);

/* ---- kernel level ---------------------------------------------------------- */
/* launch_matmul (src/kernels/matmul.h:12-13): C(M,N) = A(M,K) . B(N,K)^T
 * [+ bias(N)] [then exact-erf GELU]; fp16 in/out, fp32 accumulate.  Any
 * M, N, K >= 1; the MFMA kernels take N % 64 == 0 and K % 64 == 0, other
 * shapes go to a plain tiled kernel. */
bbh_status bbh_linear(const void *A, const void *B, void *C, int M, int N, int K,
                      const void *bias, int gelu, bbh_stream_t stream);
/* Linear + bias + residual + LayerNorm in one kernel (the fused tail of
 * attention_block / ffn_block, src/model/encoder.cu:47-50,61-64):
 * y = LN(A . B^T + bias + residual) * gamma + beta, N must be 384 and K a
 * multiple of 64.  y may alias residual.  Every pointer must be 16-byte
 * aligned (the epilogue moves residual, y, bias, gamma and beta in 16-byte
 * pieces). */
bbh_status bbh_linear_residual_layernorm(const void *A, const void *B,
                                         const void *bias, const void *residual,
                                         const void *gamma, const void *beta,
                                         void *y, int M, int N, int K, float eps,
                                         bbh_stream_t stream);
/* launch_layernorm (src/kernels/layernorm.h:6-8): y = LN(x [+ residual]).
 * Any D in [1, 4096]; y may alias x or residual. */
bbh_status bbh_layernorm(const void *x, const void *gamma, const void *beta,
                         void *y, int M, int D, float eps, const void *residual,
                         bbh_stream_t stream);
/* launch_embedding (src/kernels/embedding.h:9-12): out = word[id] +
 * pos[row % seq] + type[tt], (batch*seq, hidden) fp16. */
bbh_status bbh_embedding(const int32_t *ids, const int32_t *types,
                         const void *word, const void *pos, const void *type,
                         void *out, int seq, int hidden, int batch,
                         bbh_stream_t stream);
/* Embedding sum and the embedding LayerNorm fused (forward.cu:28-31),
 * hidden must be 384. */
bbh_status bbh_embedding_layernorm(const int32_t *ids, const int32_t *types,
                                   const void *word, const void *pos,
                                   const void *type, const void *gamma,
                                   const void *beta, void *out, int seq,
                                   int hidden, int batch, float eps,
                                   bbh_stream_t stream);
/* Masked multi-head attention straight out of the fused QKV activations:
 * launch_attention_scores + launch_softmax(mask) + launch_attention_context
 * (src/kernels/attention.h:9-18, softmax.h:11-12) as one kernel.
 * qkv (batch*seq, 3*heads*head_dim) with Q|K|V column blocks, mask
 * (batch, seq), merged (batch*seq, heads*head_dim).  head_dim must be 32,
 * seq a multiple of 16 and <= 512. */
bbh_status bbh_attention(const void *qkv, const int32_t *mask, void *merged,
                         int batch, int heads, int seq, int head_dim, float scale,
                         bbh_stream_t stream);
/* launch_attention_scores (attention.h:9-11): scores(batch*heads, seq, seq)
 * = scale * Q . K^T read strided from qkv (row stride qkv_stride, Q/K column
 * offsets q_off/k_off).  seq % 16 == 0, head_dim == 32. */
bbh_status bbh_attention_scores(const void *qkv, void *scores, int batch, int heads,
                                int seq, int head_dim, int qkv_stride, int q_off,
                                int k_off, float scale, bbh_stream_t stream);
/* launch_softmax (softmax.h:11-12): row softmax in place over (M, N); with a
 * mask, column j of row r is dropped when mask[(r / mask_stride) * N + j] ==
 * 0 (mask_stride 0: one shared mask row). */
bbh_status bbh_softmax(void *x, int M, int N, const int32_t *mask, int mask_stride,
                       bbh_stream_t stream);
/* launch_attention_context (attention.h:16-18): merged(batch*seq,
 * heads*head_dim) = probs . V, V strided from qkv at column v_off. */
bbh_status bbh_attention_context(const void *probs, const void *qkv, void *merged,
                                 int batch, int heads, int seq, int head_dim,
                                 int qkv_stride, int v_off, bbh_stream_t stream);
/* launch_mean_pool (pooling.h:9-10): out(batch, dim) = masked mean. */
bbh_status bbh_mean_pool(const void *hidden, const int32_t *mask, void *out,
                         int seq, int dim, int batch, bbh_stream_t stream);
/* launch_l2_normalize (normalize.h:7): rows of x /= max(||x||, 1e-12). */
bbh_status bbh_l2_normalize(void *x, int n, int batch, bbh_stream_t stream);
/* Masked mean pool + L2 normalize fused (forward.cu:51-52), dim 384, seq <= 512. */
bbh_status bbh_pool_normalize(const void *hidden, const int32_t *mask, void *out,
                              int seq, int dim, int batch, bbh_stream_t stream);
/* launch_gelu (src/kernels/gelu.h:9): x[i] = GELU(x[i]) in place, exact erf
 * form, n >= 0 values.  On the hot path GELU runs inside the FFN1 GEMM
 * epilogue; this entry point is the standalone operator. */
bbh_status bbh_gelu(void *x, int n, bbh_stream_t stream);

/* ---- text -> ids (WordPiece) -------------------------------------------------
 * The uncased BERT tokenizer the reference calls through sentence-transformers
 * (Hugging Face tokenizers' BertTokenizerFast, scripts/dump_weights.py:100-106,
 * scripts/dump_corpus.py:34-39, padding="max_length", truncation=True): clean
 * text, CJK ideographs split, accents stripped and text lowercased (when
 * `lowercase`), split on whitespace and punctuation, greedy longest-match
 * WordPiece with "##" continuations and [UNK] for words over 100 characters or
 * without a match.  vocab.txt holds one token per line, id = line number; it
 * must contain [CLS], [SEP], [PAD] and [UNK].  Host-side only: the outputs are
 * host arrays ready to copy to the device. */
typedef struct bbh_tokenizer bbh_tokenizer;
bbh_status bbh_tokenizer_load(const char *vocab_path, int lowercase, bbh_tokenizer **out);
bbh_status bbh_tokenizer_free(bbh_tokenizer *t);
int bbh_tokenizer_vocab_size(const bbh_tokenizer *t);
/* n NUL-terminated UTF-8 texts -> ids / types / mask, each (n, seq) int32
 * row-major: [CLS] tokens [SEP] [PAD]..., tokens truncated to seq - 2; types
 * 0; mask 1 on [CLS], tokens and [SEP].  lengths (optional, n entries) gets
 * each row's unpadded length.  Malformed UTF-8 bytes are dropped.  seq >= 2. */
bbh_status bbh_tokenize(const bbh_tokenizer *t, const char *const *texts, int n, int seq,
                        int32_t *ids, int32_t *types, int32_t *mask, int32_t *lengths);

#ifdef __cplusplus
}
#endif

#endif /* BBH_H */

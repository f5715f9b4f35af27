/*
 * rstr_hip.h -- C ABI of librstr_hip.so, the MI355X (gfx950) backend of the
 * pretrained-rstr resident continuous decode step.
 *
 * Plain pointers and sizes only.  Every call is synchronous with respect to the
 * host buffers it is given (they may be reused on return), returns 0 on
 * success or a negative RSTR_E_* status, and leaves a message readable with
 * rstr_last_error().  No exception crosses the boundary.  A session is used by
 * one host thread at a time (the reference's device-owning runtime thread,
 * src/pretrained/continuation/paged_runtime.clj:4-5); its work is ordered on
 * one in-order HIP stream, so a copy-on-write page copy issued before a step
 * is complete before that step's append (paged_attention.clj:351-353).
 *
 * Each entry cites the reference interface it replaces (file:line into the
 * reference repository).
 */
#ifndef RSTR_HIP_H
#define RSTR_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RSTR_OK 0
#define RSTR_E_INVALID -1   /* argument or descriptor validation failed      */
#define RSTR_E_HIP -2       /* a HIP runtime call failed                     */
#define RSTR_E_OOM -3       /* device or host allocation failed              */
#define RSTR_E_STATE -4     /* object closed or used out of order            */

typedef struct rstr_session rstr_session;
typedef struct rstr_model rstr_model;
typedef struct rstr_pool rstr_pool;
typedef struct rstr_decoder rstr_decoder;
typedef struct rstr_transfer rstr_transfer;

/* Descriptor flags of src/pretrained/arch/{gemma3,qwen3,llama}.clj plus the HF
 * hyper-parameters read by decoder.clj:31-56 (load-hf). */
typedef struct rstr_model_desc {
  int32_t n_layers, d_model, d_ff, n_q, n_kv, head_dim, vocab;
  int32_t weight_bits;        /* 4: Q4 block 32 + fp16 scale; 8: Q8 block 32   */
  int32_t gain_offset;        /* 1: RMSNorm gain (1 + w) (gemma3.clj:29)        */
  int32_t qk_norm;            /* per-head q/k RMSNorm                          */
  int32_t sandwich;           /* post-attention and post-FFN norms             */
  int32_t ffn_geglu;          /* 1: GELU(tanh) gate; 0: SiLU gate              */
  int32_t rope_dual;          /* local/global RoPE theta per layer            */
  int32_t global_pattern;     /* layer l is global iff (l+1) % p == 0; 0: all */
  int32_t sliding_window;     /* local-layer window in tokens; 0: none        */
  int32_t embed_scale_sqrt_d; /* embedding scaled by sqrt(d_model)            */
  float eps;                  /* RMSNorm epsilon                               */
  float attn_scale;           /* 1/sqrt(query_pre_attn_scalar or head_dim)    */
  double rope_global, rope_local;
} rstr_model_desc;

/* Tensor roles (synthetic generator keys and host-tensor binding). */
enum {
  RSTR_ROLE_EMBED = 0, RSTR_ROLE_FINAL_NORM = 1, RSTR_ROLE_ATTN_NORM = 2, RSTR_ROLE_Q = 3,
  RSTR_ROLE_K = 4, RSTR_ROLE_V = 5, RSTR_ROLE_O = 6, RSTR_ROLE_Q_NORM = 7, RSTR_ROLE_K_NORM = 8,
  RSTR_ROLE_POST_ATTN_NORM = 9, RSTR_ROLE_FFN_PRE_NORM = 10, RSTR_ROLE_FFN_POST_NORM = 11,
  RSTR_ROLE_GATE = 12, RSTR_ROLE_UP = 13, RSTR_ROLE_DOWN = 14
};

/* One host tensor as stored in a checkpoint: dtype 0 = f32, 1 = f16, 2 = bf16
 * (the SafeTensors "F32"/"F16"/"BF16" of safetensors.clj:48-72), little-endian,
 * linear weights row-major [out][in]. */
typedef struct rstr_tensor_raw {
  int32_t layer;   /* -1 for global tensors (embed, final norm) */
  int32_t role;
  int32_t dtype;
  const void* data;
  int64_t elements;
} rstr_tensor_raw;

/* One host f32 tensor: linear weights row-major [out][in] (decoder.clj:77-86). */
typedef struct rstr_tensor {
  int32_t layer;   /* -1 for global tensors (embed, final norm) */
  int32_t role;
  const float* data;
  int64_t elements;
} rstr_tensor;

/* ---- session --------------------------------------------------------------
 * Replaces raster.gpu.core/make-session (decoder_gpu.clj:1103) and
 * close-session! (continuation/model_worker.clj:35). */
int rstr_session_open(int32_t device, rstr_session** out);
int rstr_session_close(rstr_session* s);
/* Replaces ex-info messages.  Valid until the next call on the session. */
const char* rstr_last_error(const rstr_session* s);
/* Message of the last failure of an open call that returned no session. */
const char* rstr_open_error(void);
/* Free and total device memory of the session's GPU (pool sizing). */
int rstr_session_memory(rstr_session* s, int64_t* free_bytes, int64_t* total_bytes);

/* ---- model binding ----------------------------------------------------------
 * Replaces bind-decode! quantise + alloc + resident specs
 * (decoder_gpu.clj:990-1131, specs :404-475, quantisation :36-54). */
int rstr_model_bind(rstr_session* s, const rstr_model_desc* desc, const rstr_tensor* tensors,
                    int32_t n_tensors, rstr_model** out);
/* Same binding over seeded synthetic weights generated on the device
 * (N(0,0.02) linears and embedding; norm gains N(0,0.02) around the gain
 * offset, or 1+N(0,0.02)). */
int rstr_model_bind_synthetic(rstr_session* s, const rstr_model_desc* desc, uint64_t seed,
                              rstr_model** out);
/* Replaces load-hf's read-tensor-floats + quantize-stream (decoder.clj:31-56,
 * 152-189; safetensors.clj:48-152) for checkpoint tensors left in their stored
 * dtype (e.g. pointers into a memory-mapped .safetensors file): each tensor is
 * copied to the device as stored, widened to f32 there (exactly) and quantised
 * by the same device packer as rstr_model_bind, so binding from bf16 equals
 * binding the f32 widening of the same tensors. */
int rstr_model_bind_raw(rstr_session* s, const rstr_model_desc* desc, const rstr_tensor_raw* tensors,
                        int32_t n_tensors, rstr_model** out);
int rstr_model_close(rstr_model* m);
/* Device bytes of the packed linear weights streamed by one decode step. */
int64_t rstr_model_weight_bytes(const rstr_model* m);
/* Download one quantised linear in the canonical packed layout: Q4 uint8
 * [out][in/32][16] (byte j = q[2j] | q[2j+1] << 4), Q8 int8 [out][in/32][32];
 * fp16 scales [out][in/32].  Used to check bit-exact quantisation. */
int rstr_model_export_linear(rstr_model* m, int32_t layer, int32_t role, void* wq, uint16_t* ws);

/* ---- page pool --------------------------------------------------------------
 * Replaces page-pool/open-pool! device allocation (page_pool.clj:235-303):
 * fp16 key and value slabs per layer, [page][page_size][n_kv][head_dim]. */
int rstr_pool_open(rstr_model* m, int32_t page_size, int32_t physical_pages, rstr_pool** out);
int rstr_pool_close(rstr_pool* p);
/* Replaces copy-page! (page_pool.clj:892-900): one physical page of every
 * slab and layer, ordered before later work on the session stream.  Returns
 * once queued (the arguments are staged; it runs after earlier work). */
int rstr_pool_copy_page(rstr_pool* p, int32_t src_page, int32_t dst_page);
/* Raw slab transfer of fp16 elements (gpu/upload! and gpu/download on a pool
 * buffer key, page_pool.clj:284-293; the chunk restore/export staging). */
int rstr_pool_upload(rstr_pool* p, int32_t slab, int32_t layer, int64_t dst_element,
                     const uint16_t* src, int64_t elements);
int rstr_pool_download(rstr_pool* p, int32_t slab, int32_t layer, int64_t src_element,
                       uint16_t* dst, int64_t elements);
/* Synthetic N(0,1) fp16 K/V in every layer of the listed pages, keyed by
 * (seed, layer, slab, element): the stand-in for a restored prefix used by
 * throughput runs.  No reference counterpart.  Returns once queued. */
int rstr_pool_fill_synthetic(rstr_pool* p, const int32_t* pages, int32_t n_pages, uint64_t seed);

/* ---- durable chunk transfer --------------------------------------------------
 * A chunk is `token_count` consecutive tokens [start, start + token_count) of a
 * route whose logical pages are pages[0 .. n_pages).  Its payload is dense in
 * the portable layout of attention_state.clj:103-123 (payload-plan): the key
 * slab of layers 0..L-1, then the value slab of layers 0..L-1, each holding
 * token_count rows of n_kv*head_dim elements, little-endian fp16
 * (page_pool.clj:1271-1286, :chunk/version 3).  Ranges may start and end inside
 * pages and cross any physical pages; one gather or scatter kernel covers every
 * slab and layer, with one DMA copy between pinned host memory and a pool
 * staging buffer.  A submitted transfer runs on the session stream (ordered
 * after earlier steps and copies); the caller keeps `payload` alive and the
 * route's pages leased until rstr_transfer_complete, which waits, records the
 * device time and releases the transfer.  A pool with open transfers refuses
 * to close. */
typedef struct rstr_transfer_stats {
  int64_t bytes;       /* payload bytes moved between host and device       */
  float device_ms;     /* HIP events around the copy and kernel on the stream */
  int32_t direction;   /* 0 upload (restore), 1 download (export)            */
} rstr_transfer_stats;
/* Replaces submit-export-chunk! (page_pool.clj:1288-1318) and the gather of
 * export-chunk (:1347-1374): payload receives 2*L*token_count*n_kv*head_dim
 * fp16 elements on completion. */
int rstr_chunk_export_submit(rstr_pool* p, const int32_t* pages, int32_t n_pages, int32_t start,
                             int32_t token_count, uint16_t* payload, rstr_transfer** out);
/* Replaces submit-restore-chunk! (page_pool.clj:1169-1184) and restore-chunk!
 * (:1211-1224): payload_dtype 0 = fp16 elements, 1 = f32 elements rounded to
 * fp16 to nearest even (half-payload, :1084-1109). */
int rstr_chunk_restore_submit(rstr_pool* p, const int32_t* pages, int32_t n_pages, int32_t start,
                              int32_t token_count, const void* payload, int32_t payload_dtype,
                              rstr_transfer** out);
/* Replaces chunk-transfer-complete? / chunk-export-complete? (:1186-1193,
 * :1320-1327): 1 when the device work is done, 0 while pending. */
int rstr_transfer_done(rstr_transfer* t);
/* Replaces complete-restore-chunk! / complete-export-chunk! (:1195-1209,
 * :1329-1345): waits, fills `stats` (may be NULL) and frees the transfer. */
int rstr_transfer_complete(rstr_transfer* t, rstr_transfer_stats* stats);
/* Measurement only, no reference counterpart: the average device time of the
 * chunk gather (mode 0) or fp16 scatter (mode 1) kernel alone, between the pool
 * and its device staging (no host copies), over `iters` launches timed with
 * HIP events on the session stream.  Scatter overwrites the chunk's tokens
 * with whatever the staging holds. */
int rstr_chunk_bench(rstr_pool* p, const int32_t* pages, int32_t n_pages, int32_t start,
                     int32_t token_count, int32_t mode, int32_t iters, float* kernel_ms);

/* ---- paged decoder ----------------------------------------------------------
 * Replaces paged-decoder/open! (paged_decoder.clj:321-420) over a state bound
 * with :cache-mode :paged and :batch-size `batch`.  `split` is the history
 * tile (tokens, multiple of 4) of the split-K attention; it fixes the
 * attention's reduction order and so is part of the numerics contract. */
int rstr_decoder_open(rstr_model* m, rstr_pool* p, int32_t batch, int32_t pages_per_seq,
                      int32_t maxpos, int32_t split, rstr_decoder** out);
int rstr_decoder_close(rstr_decoder* d);
/* Replaces prime-lanes! -> upload-ranges! :r0 (paged_decoder.clj:462-471,
 * decoder_gpu.clj:1248-1271): the prescaled embedding of each token becomes
 * the lane's pending input row; other lanes keep their resident row.
 * Returns once queued, ordered before the next step on the session stream. */
int rstr_prime_lanes(rstr_decoder* d, int32_t n, const int32_t* lanes, const int32_t* tokens);
/* Replaces decode-row! input upload (decoder_gpu.clj:1158-1170): arbitrary
 * f32 rows [n][d_model] (the multimodal seam). */
int rstr_prime_rows(rstr_decoder* d, int32_t n, const int32_t* lanes, const float* rows);
/* Replaces step-lanes! upload-ranges! + gpu-link/run! + download :tokbuf
 * (paged_decoder.clj:562-578).  Descriptors (int32): slots[batch] (physical
 * slot page*page_size+offset, -1 = no append), row_offsets[batch+1] (0..batch),
 * positions[batch], page_table[batch*pages_per_seq] (-1 padded),
 * lengths[batch] (visible tokens including this step's row, 0 = inactive),
 * start_positions[batch].  tokens_out[batch] receives the greedy next token of
 * every lane; the next input row stays resident. */
int rstr_step_lanes(rstr_decoder* d, const int32_t* slots, const int32_t* row_offsets,
                    const int32_t* positions, const int32_t* page_table, const int32_t* lengths,
                    const int32_t* start_positions, int32_t* tokens_out);
/* No counterpart in the reference (step-lanes! is synchronous): the same step
 * without waiting for it, for callers that plan the next step while the
 * device runs this one.  Validates and copies the descriptors (same meaning
 * and errors as rstr_step_lanes), enqueues the step and returns.  At most two
 * submitted steps are in flight (a third submit fails with RSTR_E_STATE);
 * rstr_step_lanes_collect waits for the oldest one and writes its tokens.
 * Every other call on the decoder, pool or session runs after the submitted
 * steps in stream order. */
int rstr_step_lanes_submit(rstr_decoder* d, const int32_t* slots, const int32_t* row_offsets,
                           const int32_t* positions, const int32_t* page_table, const int32_t* lengths,
                           const int32_t* start_positions);
/* No counterpart in the reference: the tokens of the oldest submitted step
 * (RSTR_E_STATE when none is in flight). */
int rstr_step_lanes_collect(rstr_decoder* d, int32_t* tokens_out);
/* No counterpart in the reference: a measurement helper for the serving
 * loop's timing harness (continuation/benchmark.clj:180-194 times whole
 * step-lanes! calls).  The phases of the decoder's last rstr_step_lanes call,
 * in milliseconds: [0] descriptor validation, [1] wait for work queued before
 * the call (fills, copies, primes), [2] descriptor packing into pinned
 * staging, [3] enqueue (descriptor copy, step graph launch, token copy),
 * [4] wait for the device, [5] token hand-back, [6] the whole call, [7] the
 * device time of the step itself (HIP events around the step graph).  Writes
 * min(n, RSTR_STEP_TIMING_FIELDS) values. */
#define RSTR_STEP_TIMING_FIELDS 8
int rstr_decoder_step_timing(rstr_decoder* d, double* out, int32_t n);
/* Logits [batch][vocab] of the last step (decode-row! returning logits,
 * decoder_gpu.clj:1158-1170). */
int rstr_decode_logits(rstr_decoder* d, float* logits_out);
/* Resident input rows [batch][d_model] (the state :r0). */
int rstr_decoder_read_rows(rstr_decoder* d, float* out);
/* 1 (default): replay each step as one captured HIP graph; 0: launch eagerly. */
int rstr_decoder_set_graph(rstr_decoder* d, int32_t enabled);

/* ---- bulk paged prefill ----------------------------------------------------
 * Replaces the :prefill-T half of paged-decoder/open! (the prefill link bound
 * with :include-head-tail? false, paged_decoder.clj:380-405; per-layer
 * prefill stages decoder_gpu.clj:729-760, 1047-1053): a decoder over `rows`
 * tile rows of one route, layers only -- no head, no tail, no tokens, and the
 * decode decoder's resident input rows are left alone.  rstr_step_lanes and
 * schedules reject it. */
int rstr_prefill_open(rstr_model* m, rstr_pool* p, int32_t rows, int32_t pages_per_seq,
                      int32_t maxpos, int32_t split, rstr_decoder** out);
/* Replaces prefill-range!'s upload + gpu-link/run! (paged_decoder.clj:638-711):
 * tokens[rows], slots[rows] (the range reservation's physical slots, none -1),
 * positions[rows], the route's page_table[pages_per_seq] (-1 padded), the
 * route length (all rows included) and its start position.  Row i attends to
 * [start_position, positions[i]] and appends its K/V at slots[i]; the result
 * equals priming the same tokens one decode step at a time, bit for bit.
 * Returns when the tile's K/V are in the pool. */
int rstr_prefill_range(rstr_decoder* d, const int32_t* tokens, const int32_t* slots,
                       const int32_t* positions, const int32_t* page_table, int32_t length,
                       int32_t start_position);

/* ---- isolated routed append -------------------------------------------------
 * Replaces the paged-append runner run! (paged_append.clj:179-339) over the
 * routed append ABI (doc/serving-architecture.md:178-190): f32 rows
 * k_rows/v_rows[batch][n_kv*head_dim] -> fp16, round to nearest even, at
 * slot = page*page_size + offset; slot -1 skips the row.  Slots must be
 * distinct. */
int rstr_append_run(rstr_pool* p, int32_t layer, int32_t batch, const float* k_rows,
                    const float* v_rows, const int32_t* slots);

/* ---- isolated dequantising linear ------------------------------------------------
 * Replaces qlinear-i8 over one resident weight (decoder.clj:206-213; the GPU
 * call sites qmatmul-q4k-dp4a-rows!, decoder_gpu.clj:170-194) as a
 * kernel-level check: y[rows][n] = x W^T for int8 activations
 * xq[rows][k] with per-32-block scales xs[rows][k/32] (4-bit significands, as
 * the step's quantiser writes them), through one projection form -- 0 the
 * step's own choice, 1 the MFMA tile, 2 the one-wave weight-streaming GEMV, 3
 * its workgroup form (2 and 3 take rows <= 4) -- with the K range in `splits`
 * slices combined in the consumers' canonical tree.  Roles: RSTR_ROLE_EMBED
 * (the tied head), RSTR_ROLE_Q (the fused [q|k|v] tensor), RSTR_ROLE_O,
 * RSTR_ROLE_GATE (the fused [gate|up] tensor), RSTR_ROLE_DOWN. */
int rstr_linear_run(rstr_model* m, int32_t layer, int32_t role, int32_t rows, const int8_t* xq,
                    const float* xs, int32_t splits, int32_t form, float* y);

/* ---- isolated decode tail ------------------------------------------------------
 * Replaces decode-tail! (decoder_gpu.clj:73-78; KAT
 * decoder_gpu_composition_test.clj:9-20) with the decode step's own tail
 * kernel: per row of logits[rows][vocab] the greedy token (ties -> lowest id,
 * NaN beats every finite value, lowest NaN id), then that token's row of
 * emb[vocab][d] gathered into rows_out[rows][d]. */
int rstr_tail_run(rstr_session* s, int32_t rows, int32_t vocab, int32_t d, const float* logits,
                  const float* emb, int32_t* tokens_out, float* rows_out);

/* ---- isolated routed attention -----------------------------------------------
 * Replaces paged-attention/run! (paged_attention.clj:322-474) with f32 query
 * and output: q[batch][n_q][head_dim], one query row per sequence
 * (row_offsets 0..batch), causal visibility with window-left = window-1
 * (window 0 = none).  Reads layer `layer` of the pool. */
int rstr_attention_run(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split,
                       int32_t window, float scale, const float* q, const int32_t* row_offsets,
                       const int32_t* positions, const int32_t* page_table, int32_t pages_per_seq,
                       const int32_t* lengths, const int32_t* start_positions, float* out);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc, code that
 * must not allocate while a graph elsewhere is being captured): it is
 * allocation-free, not capturable -- it copies the host arrays in and the
 * output back with blocking copies and synchronises the session stream, so it
 * must be called outside any active stream capture.  rstr_attention_run's
 * arguments, validation, kernels and
 * results, with no hipMalloc/hipFree -- the query, descriptors, work tables,
 * split partials and output are staged in one library-owned device array of
 * RSTR_ATTN_STATIC_BYTES on each GPU (held until the process ends; its address
 * is taken when a session opens on that GPU).  A call whose staging would
 * exceed that size returns RSTR_E_INVALID before any device work.  Every call
 * on one GPU shares the array and it keeps the last call's contents, so calls
 * that overlap on one GPU (another thread, another session) race: issue them
 * from one host thread per device. */
#define RSTR_ATTN_STATIC_BYTES (64ll << 20)
int rstr_attention_run_static(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split,
                              int32_t window, float scale, const float* q, const int32_t* row_offsets,
                              const int32_t* positions, const int32_t* page_table, int32_t pages_per_seq,
                              const int32_t* lengths, const int32_t* start_positions, float* out);
/* Timing form of rstr_attention_run: inputs uploaded once, `iters` launches
 * timed with HIP events on the session stream; average ms per launch of the
 * split kernel and of the merge kernel. */
int rstr_attention_bench(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split,
                         int32_t window, float scale, const float* q, const int32_t* page_table,
                         int32_t pages_per_seq, const int32_t* lengths, int32_t iters,
                         float* split_ms, float* merge_ms);

/* ---- device-resident step schedules (measurement) ------------------------------
 * A schedule is a list of steps whose descriptors (and the synthetic prefix
 * fills and copy-on-write copies due before them) are uploaded ahead of time,
 * so a run measures device work only.  No reference counterpart; the host
 * bookkeeping that produced the descriptors is timed separately. */
typedef struct rstr_staged_step {
  const int32_t *slots, *row_offsets, *positions, *page_table, *lengths, *start_positions;
  const int32_t* fill_pages;  /* pages to fill synthetically before the step */
  int32_t n_fill;
  uint64_t fill_seed;
  const int32_t* cow_pairs;   /* (src, dst) page copies before the step */
  int32_t n_cow;
  const int32_t* prime_lanes; /* lanes primed with token embeddings before the step */
  const int32_t* prime_tokens;
  int32_t n_prime;
} rstr_staged_step;
int rstr_schedule_upload(rstr_decoder* d, const rstr_staged_step* steps, int32_t n_steps);
/* Runs staged steps [first, first+count); tokens_out[count][batch]; device_ms
 * = HIP-event time on the session stream. */
int rstr_schedule_run(rstr_decoder* d, int32_t first, int32_t count, int32_t* tokens_out,
                      float* device_ms);
/* Kernel classes timed by rstr_decoder_profile_steps (eager launches with HIP
 * events around each kernel). */
enum {
  RSTR_K_QGEMM = 0, RSTR_K_HEAD = 1, RSTR_K_ATTN_SPLIT = 2, RSTR_K_ATTN_MERGE = 3,
  RSTR_K_QKV_POST = 4, RSTR_K_ROWS = 5, RSTR_K_TAIL = 6, RSTR_K_CLASSES = 7
};
/* Runs staged steps eagerly with per-kernel events; per class: total ms and
 * launch count over the run. */
int rstr_decoder_profile_steps(rstr_decoder* d, int32_t first, int32_t count, float* class_ms,
                               int32_t* class_launches);

#ifdef __cplusplus
}
#endif
#endif

/*
 * rstr_oracle.h -- CPU restatement of the pretrained-rstr continuous decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links this library; it is
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, and only as the checker (or as the timed CPU baseline).
 *
 * What it restates (citations are into the reference repository):
 *   - decode-step op order            src/pretrained/decoder.clj:264-347
 *   - generated GPU layer/head order  src/pretrained/decoder_gpu.clj:122-220
 *   - decode tail (argmax + gather)   src/pretrained/decoder_gpu.clj:64-91
 *   - paged fp16 append               src/pretrained/continuation/paged_append.clj:44-57,
 *                                     doc/serving-architecture.md:178-190
 *   - routed paged attention          src/pretrained/continuation/paged_attention.clj:196-228,
 *                                     visibility paged_decoder.clj:166-177
 *   - lane step descriptors           src/pretrained/continuation/paged_decoder.clj:494-583
 *   - greedy argmax                   src/pretrained/sampling.clj:31-38
 *
 * The numerics inside those ops live in the reference's absent dependency
 * (org.replikativ/raster 0.2.922, deps.edn:10).  This file fixes one exact
 * definition of each (the "canonical" orders shared with the HIP kernels), so
 * the GPU path can be checked bit-for-bit.  Each function's header comment
 * says what pins it.  Functions whose rounding could only be pinned by running
 * Raster are marked "parity unpinned vs Raster".
 */
#ifndef RSTR_ORACLE_H
#define RSTR_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model descriptor: the data form of arch/{gemma3,qwen3,llama}.clj flags. */
typedef struct orc_desc {
  int32_t n_layers, d_model, d_ff, n_q, n_kv, head_dim, vocab;
  int32_t weight_bits;        /* 4 = Q4 block-32 fp16 scale, 8 = Q8 block-32 */
  int32_t gain_offset;        /* 1: (1+w) RMSNorm gain (gemma3.clj:29)       */
  int32_t qk_norm;            /* per-head q/k RMSNorm                         */
  int32_t sandwich;           /* post-attn + post-ffn norms                   */
  int32_t ffn_geglu;          /* 1 = GELU(tanh) gate, 0 = SiLU gate           */
  int32_t rope_dual;          /* local/global theta per layer                 */
  int32_t global_pattern;     /* layer l global iff (l+1)%p==0; 0 = all       */
  int32_t sliding_window;     /* tokens; 0 = none                             */
  int32_t embed_scale_sqrt_d; /* embedding multiplied by sqrt(d_model)        */
  float eps;
  float attn_scale;
  double rope_global, rope_local;
} orc_desc;

/* Tensor roles of the synthetic weight generator (key = f(seed, layer, role)). */
enum {
  ORC_ROLE_EMBED = 0, ORC_ROLE_FINAL_NORM = 1, ORC_ROLE_ATTN_NORM = 2, ORC_ROLE_Q = 3,
  ORC_ROLE_K = 4, ORC_ROLE_V = 5, ORC_ROLE_O = 6, ORC_ROLE_Q_NORM = 7, ORC_ROLE_K_NORM = 8,
  ORC_ROLE_POST_ATTN_NORM = 9, ORC_ROLE_FFN_PRE_NORM = 10, ORC_ROLE_FFN_POST_NORM = 11,
  ORC_ROLE_GATE = 12, ORC_ROLE_UP = 13, ORC_ROLE_DOWN = 14
};

/* ---- scalar numerics ---------------------------------------------------- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
float orc_exp(float x);
float orc_gelu_tanh(float g);
float orc_silu(float g);
uint64_t orc_splitmix64(uint64_t x);
uint64_t orc_tensor_key(uint64_t seed, int32_t layer, int32_t role);
float orc_normal(uint64_t key, uint64_t index, double mean, double std);
void orc_normal_fill(uint64_t key, uint64_t start, int64_t n, double mean, double std, float* out);

/* ---- block quantisation ------------------------------------------------- */
void orc_quant_q4(const float* w, int64_t rows, int64_t cols, uint8_t* nib, uint16_t* scales);
void orc_quant_q8(const float* w, int64_t rows, int64_t cols, int8_t* q, uint16_t* scales);
float orc_act_scale(float amax);
void orc_set_act_scale_plain(int32_t on);   /* measurement hook: plain RN(amax/127) */
void orc_quant_act(const float* x, int32_t rows, int32_t cols, int8_t* q, float* scales);
void orc_qlinear(int32_t bits, const void* wq, const uint16_t* ws, int32_t n_out, int32_t k_in,
                 const int8_t* xq, const float* xs, int32_t rows, float* y);

/* ---- row ops ------------------------------------------------------------ */
float orc_sumsq(const float* x, int32_t n);
void orc_rmsnorm(const float* x, const float* g, float gain_offset, float eps, int32_t rows,
                 int32_t n, float* y);
void orc_rope_table(double theta, int32_t head_dim, int32_t maxpos, float* cos_t, float* sin_t);
void orc_rope(const float* x, int32_t rows, int32_t heads, int32_t head_dim, const int32_t* pos,
              const float* cos_t, const float* sin_t, float* y);
float orc_dot_canon(const float* q, const void* k, int32_t k_f16, int32_t hd);
void orc_attention(const float* q, const void* kpages, const void* vpages, int32_t kv_f16,
                   int32_t page_size, int32_t n_kv, int32_t hd, int32_t n_q, int32_t batch,
                   const int32_t* page_table, int32_t pps, const int32_t* lengths, int32_t window,
                   float scale, int32_t split, float* out);
void orc_argmax_rows(const float* logits, int32_t rows, int32_t vocab, int32_t* out);

/* ---- model + paged decoder ---------------------------------------------- */
typedef struct orc_model orc_model;
typedef struct orc_decoder orc_decoder;

orc_model* orc_model_synthetic(const orc_desc* desc, uint64_t seed);
void orc_model_free(orc_model* m);
/* Replace one tensor by host f32 values (linears/embedding quantised, norms copied). */
int32_t orc_model_set_tensor(orc_model* m, int32_t layer, int32_t role, const float* src, int64_t n);
/* Canonical packed bytes of one linear tensor (role, layer); returns bytes written. */
int64_t orc_model_tensor(const orc_model* m, int32_t layer, int32_t role, void* wq, uint16_t* ws);
/* f32 gain vector of a norm role; returns elements. */
int64_t orc_model_norm(const orc_model* m, int32_t layer, int32_t role, float* out);
void orc_embed_row(const orc_model* m, int32_t token, float* out);

orc_decoder* orc_decoder_open(const orc_model* m, int32_t batch, int32_t page_size,
                              int32_t physical_pages, int32_t pages_per_seq, int32_t maxpos,
                              int32_t kv_f16, int32_t split);
void orc_decoder_free(orc_decoder* d);
void orc_prime_lanes(orc_decoder* d, int32_t n, const int32_t* lanes, const int32_t* tokens);
void orc_prime_rows(orc_decoder* d, int32_t n, const int32_t* lanes, const float* rows);
int32_t orc_step_lanes(orc_decoder* d, const int32_t* slots, const int32_t* row_offsets,
                       const int32_t* positions, const int32_t* page_table,
                       const int32_t* lengths, const int32_t* start_positions,
                       int32_t* tokens_out);
const float* orc_logits(const orc_decoder* d);
const float* orc_r0(const orc_decoder* d);
void orc_copy_page(orc_decoder* d, int32_t src, int32_t dst);
void orc_fill_synthetic(orc_decoder* d, int32_t page, uint64_t seed);
/* Raw page-slab access: slab 0 = key, 1 = value.  Element type is fp16 bits or f32. */
void* orc_slab(orc_decoder* d, int32_t slab, int32_t layer);
const char* orc_last_error(void);
int orc_num_threads(void);
double orc_stream_triad(int64_t n, int32_t reps);

#ifdef __cplusplus
}
#endif
#endif

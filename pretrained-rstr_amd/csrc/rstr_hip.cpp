// rstr_hip.cpp -- C ABI of the MI355X resident continuous decode step.
//
// Host side of librstr_hip.so: sessions, resident model binding, the fp16 page
// pool, the paged lane decoder (descriptor validation, upload, one HIP-graph
// replay per step, token download), the isolated routed attention and the
// device-resident schedules used for measurement.  The op sequence of a step
// follows the reference's linked paged executable: per layer the generated
// pre stage, routed append, routed attention and post stage, then head and
// tail (src/pretrained/continuation/paged_decoder.clj:179-319,
// src/pretrained/decoder_gpu.clj:122-220).
#include "../../include/rstr_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "device_math.h"
#include "kernels.h"

using namespace rstr;

static thread_local std::string g_open_err;

struct rstr_session {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  void* scratch = nullptr;  // device address of this GPU's static staging array
};

static_assert(RSTR_ATTN_STATIC_BYTES == RSTR_STATIC_SCRATCH_BYTES, "one staging size in the ABI and the kernels");

namespace {

int fail(rstr_session* s, int code, const std::string& msg) {
  if (s) s->err = msg;
  else g_open_err = msg;
  return code;
}

#define HIPCHK(S, expr)                                                                  \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess)                                                                \
      return fail((S), e_ == hipErrorOutOfMemory ? RSTR_E_OOM : RSTR_E_HIP,              \
                  std::string(#expr) + ": " + hipGetErrorString(e_));                    \
  } while (0)

template <class T>
hipError_t dmalloc(T** p, size_t elems) {
  *p = nullptr;
  if (elems == 0) elems = 1;
  return hipMalloc((void**)p, elems * sizeof(T));
}

inline int64_t linear_bytes(int bits, int n, int k) { return (int64_t)n * k / 32 * (bits == 4 ? 16 : 32); }

bool global_layer(const rstr_model_desc& d, int l) {
  if (d.global_pattern <= 0) return true;
  return ((l + 1) % d.global_pattern) == 0;
}

}  // namespace

struct LayerW {
  QTensor qkv, o, gu, down;
  float *attn_norm = nullptr, *ffn_pre_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  float *post_attn_norm = nullptr, *ffn_post_norm = nullptr;
};

struct rstr_model {
  rstr_session* s = nullptr;
  rstr_model_desc d{};
  std::vector<LayerW> layers;
  QTensor head;
  float* final_norm = nullptr;
  float* emb = nullptr;  // prescaled f32 [vocab][d]
  std::vector<void*> allocs;
  int64_t weight_bytes = 0;
};

// Pinned host staging for the small int32 lists that page fills, page copies
// and primes send to the device: a ring of slots, each reused only after its
// previous copy has run (an event per slot).  A call returns once its
// arguments are staged and its work is queued on the session's stream, so it
// does not wait for steps submitted before it.
struct HostRing {
  static constexpr int N = 8;
  int32_t* h[N] = {};
  size_t cap[N] = {};
  hipEvent_t ev[N] = {};
  bool used[N] = {};
  int next = 0;
  // copy a[0..na) then b[0..nb) into a free slot
  hipError_t stage(const int32_t* a, size_t na, const int32_t* b, size_t nb, int32_t** out, int* slot) {
    const int k = next;
    next = (next + 1) % N;
    hipError_t e = hipSuccess;
    if (used[k] && (e = hipEventSynchronize(ev[k])) != hipSuccess) return e;
    used[k] = false;
    if (!ev[k] && (e = hipEventCreateWithFlags(&ev[k], hipEventDisableTiming)) != hipSuccess) return e;
    if (cap[k] < na + nb) {
      if (h[k]) hipHostFree(h[k]);
      h[k] = nullptr;
      cap[k] = 0;
      if ((e = hipHostMalloc((void**)&h[k], sizeof(int32_t) * std::max<size_t>(na + nb, 64))) != hipSuccess) return e;
      cap[k] = std::max<size_t>(na + nb, 64);
    }
    if (na) std::memcpy(h[k], a, sizeof(int32_t) * na);
    if (nb) std::memcpy(h[k] + na, b, sizeof(int32_t) * nb);
    *out = h[k];
    *slot = k;
    return hipSuccess;
  }
  // the slot's copies are queued: it is free again once the stream passes here
  hipError_t queued(int slot, hipStream_t st) {
    used[slot] = true;
    return hipEventRecord(ev[slot], st);
  }
  void release() {
    for (int k = 0; k < N; k++) {
      if (h[k]) hipHostFree(h[k]);
      if (ev[k]) hipEventDestroy(ev[k]);
      h[k] = nullptr;
      ev[k] = nullptr;
    }
  }
};

struct rstr_pool {
  rstr_model* m = nullptr;
  int page_size = 0, physical_pages = 0;
  int64_t page_elems = 0;                 // page_size * n_kv * head_dim
  std::vector<uint16_t*> slabs;           // [K0..K{L-1}, V0..V{L-1}]
  uint16_t** d_slabs = nullptr;
  int32_t* d_pairs = nullptr;
  int32_t* h_pairs = nullptr;             // pinned
  HostRing ring;                          // staging of fill page lists and copy pairs
  int32_t* d_fill = nullptr;              // page list of a synthetic fill
  int fill_cap = 0;
  uint16_t* tmpl = nullptr;               // synthetic-prefix page templates
  uint64_t tmpl_seed = 0;
  bool tmpl_ready = false;
  // durable chunk transfers: dense payload staging and the route's page list
  void* stage = nullptr;
  size_t stage_bytes = 0;
  int32_t* d_chunk_pages = nullptr;
  int chunk_pages_cap = 0;
  int open_transfers = 0;
  std::vector<std::pair<void*, size_t>> pinned;  // idle pinned transfer buffers, reused
};

struct rstr_transfer {
  rstr_pool* p = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  void* host = nullptr;          // pinned: page list, then the payload
  size_t host_bytes = 0;
  uint16_t* user_dst = nullptr;  // export destination
  size_t payload_bytes = 0;
  size_t host_payload_offset = 0;
  int direction = 0;             // 0 restore (upload), 1 export (download)
};

// Generate (once per seed) the page templates the synthetic fill copies from.
static hipError_t ensure_templates(rstr_pool* p, uint64_t seed) {
  if (p->tmpl_ready && p->tmpl_seed == seed) return hipSuccess;
  int L = p->m->d.n_layers;
  if (!p->tmpl) {
    hipError_t e = hipMalloc(&p->tmpl, sizeof(uint16_t) * (size_t)2 * L * RSTR_SYNTH_TEMPLATES * p->page_elems);
    if (e != hipSuccess) return e;
  }
  hipError_t e = launch_gen_templates(p->m->s->stream, p->tmpl, L, p->page_elems, seed);
  if (e == hipSuccess) e = hipStreamSynchronize(p->m->s->stream);
  if (e == hipSuccess) {
    p->tmpl_seed = seed;
    p->tmpl_ready = true;
  }
  return e;
}

struct StagedDev {                        // one uploaded schedule step
  int64_t desc_off;                       // int32 offset in sched_desc
  int64_t fill_off;
  int32_t n_fill;
  uint64_t fill_seed;
  int64_t cow_off;
  int32_t n_cow;
  int64_t prime_off;
  int32_t n_prime;
  bool fused;                             // qkv post-processing inside attention (see rstr_decoder)
};

struct rstr_decoder {
  rstr_model* m = nullptr;
  rstr_pool* p = nullptr;
  int B = 0, pps = 0, maxpos = 0, split = 0, mpad = 0, kmax = 0, max_items = 0;
  int qd = 0, kvr = 0, nqkv = 0;
  int s_qkv = 1, s_o = 1, s_gu = 1, s_down = 1;   // split-K slices per projection
  // device state / scratch
  float *r0 = nullptr, *xmid = nullptr, *o = nullptr, *yqkv = nullptr, *qr = nullptr;
  float *gu = nullptr, *logits = nullptr, *part = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;   // [2][maxpos][hd/2]
  ActBuf act;
  ActBuf act_ff;                                    // down-projection input when gate/up fuses the activation
  bool fuse_act = false;
  // qkv post-processing (qk-norm, RoPE, K/V append) inside the few-item
  // attention kernel, for steps where no lane's visible range holds another
  // lane's appended slot (`mark`: scratch of that check, one word per page)
  bool fuse_qkv = false;
  // every lane's visible range is one attention split (maxpos <= split) and the
  // few-item kernel runs: it writes the quantised attention output itself and
  // the step has no merge launch
  bool attn_direct = false;
  std::vector<int32_t> mark;
  int32_t* desc = nullptr;                          // device descriptors
  int32_t* lane_tab = nullptr;                      // [2][tabw] attention work tables
  size_t tabw = 0;                                  // words per work table
  int32_t* tokbuf = nullptr;
  int32_t* amax_cand = nullptr;  // tail candidates, 2 words per (row, segment)
  int32_t *d_lanes = nullptr, *d_tokens = nullptr;  // priming staging
  // pinned host staging
  int32_t* h_desc = nullptr;
  int32_t* h_tok = nullptr;
  int64_t desc_words = 0;
  // offsets into desc
  int64_t off_slots = 0, off_rows = 0, off_pos = 0, off_len = 0, off_start = 0, off_pt = 0;
  bool use_graph = true;
  bool head_tail = true;                            // false: bulk-prefill decoder (layers only)
  hipGraphExec_t graph = nullptr;
  // schedules
  int32_t* sched_desc = nullptr;
  int32_t* sched_pages = nullptr;
  int32_t* sched_tok = nullptr;
  std::vector<StagedDev> sched;
  int64_t sched_desc_cap = 0, sched_pages_cap = 0, sched_tok_cap = 0;
  bool has_logits = false;
  // phases of the last rstr_step_lanes call (rstr_decoder_step_timing)
  hipEvent_t ev_step[2] = {nullptr, nullptr};
  double step_ms[RSTR_STEP_TIMING_FIELDS] = {};
  // steps submitted without waiting (rstr_step_lanes_submit / _collect): two
  // pinned descriptor and token slots, the in-flight steps in submission order
  int32_t* h_desc_q[2] = {nullptr, nullptr};
  int32_t* h_tok_q[2] = {nullptr, nullptr};
  hipEvent_t ev_q[2] = {nullptr, nullptr};
  int q_first = 0, q_n = 0;
  HostRing ring;  // staging of primed lanes and tokens
};

// ---------------------------------------------------------------------------
// session
// ---------------------------------------------------------------------------
extern "C" int rstr_session_open(int32_t device, rstr_session** out) {
  if (!out) return fail(nullptr, RSTR_E_INVALID, "null output pointer");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(nullptr, RSTR_E_HIP, "no HIP device available");
  if (device < 0 || device >= n) return fail(nullptr, RSTR_E_INVALID, "device id out of range");
  if (hipSetDevice(device) != hipSuccess) return fail(nullptr, RSTR_E_HIP, "hipSetDevice failed");
  auto s = new rstr_session();
  s->device = device;
  if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) {
    delete s;
    return fail(nullptr, RSTR_E_HIP, "hipStreamCreate failed");
  }
  // the allocation-free entry's staging array of this GPU (its address differs per GPU)
  hipError_t se = static_scratch_address(&s->scratch);
  if (se != hipSuccess || !s->scratch) {
    hipStreamDestroy(s->stream);
    delete s;
    return fail(nullptr, RSTR_E_HIP, std::string("static staging address: ") + hipGetErrorString(se));
  }
  *out = s;
  return RSTR_OK;
}

extern "C" int rstr_session_close(rstr_session* s) {
  if (!s) return RSTR_OK;
  hipSetDevice(s->device);
  hipStreamSynchronize(s->stream);
  hipStreamDestroy(s->stream);
  delete s;
  return RSTR_OK;
}

extern "C" const char* rstr_last_error(const rstr_session* s) { return s ? s->err.c_str() : ""; }

extern "C" int rstr_session_memory(rstr_session* s, int64_t* free_bytes, int64_t* total_bytes) {
  if (!s) return fail(nullptr, RSTR_E_INVALID, "null session");
  HIPCHK(s, hipSetDevice(s->device));
  size_t f = 0, t = 0;
  HIPCHK(s, hipMemGetInfo(&f, &t));
  if (free_bytes) *free_bytes = (int64_t)f;
  if (total_bytes) *total_bytes = (int64_t)t;
  return RSTR_OK;
}
extern "C" const char* rstr_open_error(void) { return g_open_err.c_str(); }

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
static int validate_desc(rstr_session* s, const rstr_model_desc* d) {
  if (!d) return fail(s, RSTR_E_INVALID, "null model descriptor");
  if (d->n_layers <= 0 || d->d_model <= 0 || d->d_ff <= 0 || d->n_q <= 0 || d->n_kv <= 0 ||
      d->head_dim <= 0 || d->vocab <= 0)
    return fail(s, RSTR_E_INVALID, "model dimensions must be positive");
  if (d->weight_bits != 4 && d->weight_bits != 8)
    return fail(s, RSTR_E_INVALID, "weight_bits must be 4 or 8");
  if (d->n_q % d->n_kv) return fail(s, RSTR_E_INVALID, "n_q must be a multiple of n_kv");
  if (d->head_dim != 64 && d->head_dim != 128 && d->head_dim != 256)
    return fail(s, RSTR_E_INVALID, "head_dim must be 64, 128 or 256");
  int g = d->n_q / d->n_kv;
  if (g != 1 && g != 2 && g != 4 && g != 8)
    return fail(s, RSTR_E_INVALID, "GQA group n_q/n_kv must be 1, 2, 4 or 8");
  int qd = d->n_q * d->head_dim, kvr = d->n_kv * d->head_dim;
  for (int k : {d->d_model, qd, d->d_ff})
    if (k % 128) return fail(s, RSTR_E_INVALID, "projection input widths must be multiples of 128");
  for (int n : {qd, kvr, d->d_model, d->d_ff, d->vocab})
    if (n % 16) return fail(s, RSTR_E_INVALID, "projection output widths must be multiples of 16");
  if (d->sliding_window < 0) return fail(s, RSTR_E_INVALID, "sliding window must be >= 0");
  return RSTR_OK;
}

static int alloc_q(rstr_model* m, QTensor& t, int n, int k) {
  t.n = n;
  t.k = k;
  t.bits = m->d.weight_bits;
  int64_t wb = linear_bytes(t.bits, n, k);
  HIPCHK(m->s, hipMalloc(&t.w, (size_t)wb));
  m->allocs.push_back(t.w);
  HIPCHK(m->s, dmalloc(&t.s, (size_t)n * (k / 32)));
  m->allocs.push_back(t.s);
  m->weight_bytes += wb + (int64_t)n * (k / 32) * 2;
  return RSTR_OK;
}

static int alloc_f(rstr_model* m, float** p, int64_t n) {
  HIPCHK(m->s, dmalloc(p, (size_t)n));
  m->allocs.push_back(*p);
  return RSTR_OK;
}

static int model_alloc(rstr_model* m) {
  const auto& d = m->d;
  int qd = d.n_q * d.head_dim, kvr = d.n_kv * d.head_dim;
  m->layers.resize(d.n_layers);
  int rc;
  for (auto& L : m->layers) {
    if ((rc = alloc_q(m, L.qkv, qd + 2 * kvr, d.d_model))) return rc;
    if ((rc = alloc_q(m, L.o, d.d_model, qd))) return rc;
    if ((rc = alloc_q(m, L.gu, 2 * d.d_ff, d.d_model))) return rc;
    if ((rc = alloc_q(m, L.down, d.d_model, d.d_ff))) return rc;
    if ((rc = alloc_f(m, &L.attn_norm, d.d_model))) return rc;
    if ((rc = alloc_f(m, &L.ffn_pre_norm, d.d_model))) return rc;
    if (d.qk_norm) {
      if ((rc = alloc_f(m, &L.q_norm, d.head_dim))) return rc;
      if ((rc = alloc_f(m, &L.k_norm, d.head_dim))) return rc;
    }
    if (d.sandwich) {
      if ((rc = alloc_f(m, &L.post_attn_norm, d.d_model))) return rc;
      if ((rc = alloc_f(m, &L.ffn_post_norm, d.d_model))) return rc;
    }
  }
  if ((rc = alloc_q(m, m->head, d.vocab, d.d_model))) return rc;
  if ((rc = alloc_f(m, &m->final_norm, d.d_model))) return rc;
  if ((rc = alloc_f(m, &m->emb, (int64_t)d.vocab * d.d_model))) return rc;
  return RSTR_OK;
}

static void model_free(rstr_model* m) {
  if (!m) return;
  hipSetDevice(m->s->device);
  for (void* p : m->allocs) hipFree(p);
  delete m;
}

// Where each linear role lives in the concatenated device tensors.
static bool linear_slot(rstr_model* m, int layer, int role, QTensor** t, int* col_off, int* n,
                        int* k) {
  const auto& d = m->d;
  int qd = d.n_q * d.head_dim, kvr = d.n_kv * d.head_dim;
  if (role == RSTR_ROLE_EMBED) {
    *t = &m->head; *col_off = 0; *n = d.vocab; *k = d.d_model;
    return true;
  }
  if (layer < 0 || layer >= d.n_layers) return false;
  LayerW& L = m->layers[layer];
  switch (role) {
    case RSTR_ROLE_Q: *t = &L.qkv; *col_off = 0; *n = qd; *k = d.d_model; return true;
    case RSTR_ROLE_K: *t = &L.qkv; *col_off = qd; *n = kvr; *k = d.d_model; return true;
    case RSTR_ROLE_V: *t = &L.qkv; *col_off = qd + kvr; *n = kvr; *k = d.d_model; return true;
    case RSTR_ROLE_O: *t = &L.o; *col_off = 0; *n = d.d_model; *k = qd; return true;
    case RSTR_ROLE_GATE: *t = &L.gu; *col_off = 0; *n = d.d_ff; *k = d.d_model; return true;
    case RSTR_ROLE_UP: *t = &L.gu; *col_off = d.d_ff; *n = d.d_ff; *k = d.d_model; return true;
    case RSTR_ROLE_DOWN: *t = &L.down; *col_off = 0; *n = d.d_model; *k = d.d_ff; return true;
    default: return false;
  }
}

static float* norm_slot(rstr_model* m, int layer, int role, int* n) {
  const auto& d = m->d;
  *n = d.d_model;
  if (role == RSTR_ROLE_FINAL_NORM) return m->final_norm;
  if (layer < 0 || layer >= d.n_layers) return nullptr;
  LayerW& L = m->layers[layer];
  switch (role) {
    case RSTR_ROLE_ATTN_NORM: return L.attn_norm;
    case RSTR_ROLE_FFN_PRE_NORM: return L.ffn_pre_norm;
    case RSTR_ROLE_POST_ATTN_NORM: return L.post_attn_norm;
    case RSTR_ROLE_FFN_POST_NORM: return L.ffn_post_norm;
    case RSTR_ROLE_Q_NORM: *n = d.head_dim; return L.q_norm;
    case RSTR_ROLE_K_NORM: *n = d.head_dim; return L.k_norm;
    default: return nullptr;
  }
}

static const int kLinearRoles[] = {RSTR_ROLE_Q, RSTR_ROLE_K, RSTR_ROLE_V, RSTR_ROLE_O,
                                   RSTR_ROLE_GATE, RSTR_ROLE_UP, RSTR_ROLE_DOWN};

static int model_generate(rstr_model* m, uint64_t seed) {
  const auto& d = m->d;
  hipStream_t st = m->s->stream;
  double nmean = d.gain_offset ? 0.0 : 1.0;
  for (int l = 0; l < d.n_layers; l++) {
    for (int role : kLinearRoles) {
      QTensor* t; int off, n, k;
      linear_slot(m, l, role, &t, &off, &n, &k);
      HIPCHK(m->s, launch_gen_linear(st, *t, off, n, k, tensor_key(seed, l, role), nullptr));
    }
    for (int role : {RSTR_ROLE_ATTN_NORM, RSTR_ROLE_FFN_PRE_NORM, RSTR_ROLE_Q_NORM, RSTR_ROLE_K_NORM,
                     RSTR_ROLE_POST_ATTN_NORM, RSTR_ROLE_FFN_POST_NORM}) {
      int n;
      float* g = norm_slot(m, l, role, &n);
      if (g) HIPCHK(m->s, launch_gen_f32(st, g, n, tensor_key(seed, l, role), nmean, 0.02, 1.0));
    }
  }
  uint64_t ek = tensor_key(seed, -1, RSTR_ROLE_EMBED);
  HIPCHK(m->s, launch_gen_linear(st, m->head, 0, d.vocab, d.d_model, ek, nullptr));
  double scale = d.embed_scale_sqrt_d ? std::sqrt((double)d.d_model) : 1.0;
  HIPCHK(m->s, launch_gen_f32(st, m->emb, (int64_t)d.vocab * d.d_model, ek, 0.0, 0.02, scale));
  HIPCHK(m->s, launch_gen_f32(st, m->final_norm, d.d_model, tensor_key(seed, -1, RSTR_ROLE_FINAL_NORM),
                              nmean, 0.02, 1.0));
  HIPCHK(m->s, hipStreamSynchronize(st));
  return RSTR_OK;
}

static int model_begin(rstr_session* s, const rstr_model_desc* desc, rstr_model** out,
                       rstr_model** mm) {
  if (!s) return fail(nullptr, RSTR_E_INVALID, "null session");
  if (!out) return fail(s, RSTR_E_INVALID, "null output pointer");
  *out = nullptr;
  int rc = validate_desc(s, desc);
  if (rc) return rc;
  HIPCHK(s, hipSetDevice(s->device));
  auto m = new rstr_model();
  m->s = s;
  m->d = *desc;
  if ((rc = model_alloc(m))) {
    model_free(m);
    return rc;
  }
  *mm = m;
  return RSTR_OK;
}

extern "C" int rstr_model_bind_synthetic(rstr_session* s, const rstr_model_desc* desc, uint64_t seed,
                                         rstr_model** out) {
  rstr_model* m = nullptr;
  int rc = model_begin(s, desc, out, &m);
  if (rc) return rc;
  if ((rc = model_generate(m, seed))) {
    model_free(m);
    return rc;
  }
  *out = m;
  return RSTR_OK;
}

// Bind host tensors of f32 (0), f16 (1) or bf16 (2) elements: each is uploaded
// as stored, widened to f32 on the device and quantised there.
static int bind_tensors(rstr_session* s, const rstr_model_desc* desc, int32_t n_tensors,
                        const rstr_tensor_raw* tensors, rstr_model** out) {
  rstr_model* m = nullptr;
  int rc = model_begin(s, desc, out, &m);
  if (rc) return rc;
  const auto& d = m->d;
  hipStream_t st = s->stream;
  // every tensor the flags require must be present exactly once
  std::vector<char> seen((size_t)(d.n_layers + 1) * 16, 0);
  float* tmp = nullptr;
  void* raw = nullptr;
  size_t tmp_cap = 0, raw_cap = 0;
  auto bail = [&](int code, const std::string& msg) {
    if (tmp) hipFree(tmp);
    if (raw) hipFree(raw);
    model_free(m);
    return fail(s, code, msg);
  };
  for (int32_t i = 0; i < n_tensors; i++) {
    const rstr_tensor_raw& t = tensors[i];
    if (!t.data) return bail(RSTR_E_INVALID, "tensor without data");
    if (t.dtype < 0 || t.dtype > 2) return bail(RSTR_E_INVALID, "Unsupported dtype");
    int li = t.layer + 1;
    if (li < 0 || li > d.n_layers || t.role < 0 || t.role > 14)
      return bail(RSTR_E_INVALID, "tensor layer or role out of range");
    if (seen[(size_t)li * 16 + t.role]) return bail(RSTR_E_INVALID, "duplicate tensor");
    seen[(size_t)li * 16 + t.role] = 1;
    QTensor* q; int off, n, k;
    const bool linear = linear_slot(m, t.layer, t.role, &q, &off, &n, &k) != 0;
    int n2 = 0;
    float* g = linear ? nullptr : norm_slot(m, t.layer, t.role, &n2);
    if (!linear && !g) return bail(RSTR_E_INVALID, "tensor role not used by this descriptor");
    const size_t need = linear ? (size_t)n * k : (size_t)n2;
    if ((size_t)t.elements != need)
      return bail(RSTR_E_INVALID, linear ? "linear tensor size mismatch" : "norm tensor size mismatch");
    const size_t esz = t.dtype == 0 ? 4 : 2;
    if (need > tmp_cap) {
      if (tmp) hipFree(tmp);
      tmp = nullptr;
      if (hipMalloc(&tmp, need * sizeof(float)) != hipSuccess) return bail(RSTR_E_OOM, "hipMalloc");
      tmp_cap = need;
    }
    if (t.dtype == 0) {
      if (hipMemcpy(tmp, t.data, need * 4, hipMemcpyHostToDevice) != hipSuccess)
        return bail(RSTR_E_HIP, "weight upload failed");
    } else {
      if (need * esz > raw_cap) {
        if (raw) hipFree(raw);
        raw = nullptr;
        if (hipMalloc(&raw, need * esz) != hipSuccess) return bail(RSTR_E_OOM, "hipMalloc");
        raw_cap = need * esz;
      }
      if (hipMemcpy(raw, t.data, need * esz, hipMemcpyHostToDevice) != hipSuccess ||
          launch_widen(st, t.dtype, raw, tmp, (int64_t)need) != hipSuccess)
        return bail(RSTR_E_HIP, "weight upload failed");
    }
    if (linear) {
      if (launch_gen_linear(st, *q, off, n, k, 0, tmp) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
        return bail(RSTR_E_HIP, "weight quantisation failed");
      if (t.role == RSTR_ROLE_EMBED) {
        double scale = d.embed_scale_sqrt_d ? std::sqrt((double)d.d_model) : 1.0;
        if (launch_prescale(st, m->emb, tmp, (int64_t)n * k, scale) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
          return bail(RSTR_E_HIP, "embedding prescale failed");
      }
    } else if (hipMemcpyAsync(g, tmp, sizeof(float) * n2, hipMemcpyDeviceToDevice, st) != hipSuccess ||
               hipStreamSynchronize(st) != hipSuccess) {
      return bail(RSTR_E_HIP, "norm upload failed");
    }
  }
  if (tmp) hipFree(tmp);
  if (raw) hipFree(raw);
  tmp = nullptr;
  raw = nullptr;
  auto need = [&](int layer, int role) { return seen[(size_t)(layer + 1) * 16 + role] != 0; };
  bool ok = need(-1, RSTR_ROLE_EMBED) && need(-1, RSTR_ROLE_FINAL_NORM);
  for (int l = 0; l < d.n_layers && ok; l++) {
    for (int role : kLinearRoles) ok = ok && need(l, role);
    ok = ok && need(l, RSTR_ROLE_ATTN_NORM) && need(l, RSTR_ROLE_FFN_PRE_NORM);
    if (d.qk_norm) ok = ok && need(l, RSTR_ROLE_Q_NORM) && need(l, RSTR_ROLE_K_NORM);
    if (d.sandwich) ok = ok && need(l, RSTR_ROLE_POST_ATTN_NORM) && need(l, RSTR_ROLE_FFN_POST_NORM);
  }
  if (!ok) {
    model_free(m);
    return fail(s, RSTR_E_INVALID, "a tensor required by the descriptor is missing");
  }
  *out = m;
  return RSTR_OK;
}

extern "C" int rstr_model_bind(rstr_session* s, const rstr_model_desc* desc, const rstr_tensor* tensors,
                               int32_t n_tensors, rstr_model** out) {
  if (n_tensors < 0 || (n_tensors && !tensors)) return fail(s, RSTR_E_INVALID, "invalid tensor list");
  std::vector<rstr_tensor_raw> raw((size_t)n_tensors);
  for (int32_t i = 0; i < n_tensors; i++)
    raw[i] = rstr_tensor_raw{tensors[i].layer, tensors[i].role, 0, tensors[i].data, tensors[i].elements};
  return bind_tensors(s, desc, n_tensors, raw.data(), out);
}

extern "C" int rstr_model_bind_raw(rstr_session* s, const rstr_model_desc* desc, const rstr_tensor_raw* tensors,
                                   int32_t n_tensors, rstr_model** out) {
  if (n_tensors < 0 || (n_tensors && !tensors)) return fail(s, RSTR_E_INVALID, "invalid tensor list");
  return bind_tensors(s, desc, n_tensors, tensors, out);
}

extern "C" int rstr_model_close(rstr_model* m) {
  if (!m) return RSTR_OK;
  hipSetDevice(m->s->device);
  hipStreamSynchronize(m->s->stream);
  model_free(m);
  return RSTR_OK;
}

extern "C" int64_t rstr_model_weight_bytes(const rstr_model* m) { return m ? m->weight_bytes : -1; }

extern "C" int rstr_model_export_linear(rstr_model* m, int32_t layer, int32_t role, void* wq,
                                        uint16_t* ws) {
  if (!m) return fail(nullptr, RSTR_E_INVALID, "null model");
  rstr_session* s = m->s;
  QTensor* t; int off, n, k;
  if (!linear_slot(m, layer, role, &t, &off, &n, &k)) return fail(s, RSTR_E_INVALID, "not a linear role");
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  int bits = t->bits, nb = k / 32, nb4 = nb / 4, DW = bits == 4 ? 1 : 2;
  int ct0 = off / 16, nct = n / 16;
  size_t wdw = (size_t)nct * nb4 * 256 * DW, sw = (size_t)nct * nb4 * 64;
  std::vector<uint32_t> hw(wdw);
  std::vector<uint16_t> hs(sw);
  HIPCHK(s, hipMemcpy(hw.data(), (uint32_t*)t->w + (size_t)ct0 * nb4 * 256 * DW, wdw * 4,
                      hipMemcpyDeviceToHost));
  HIPCHK(s, hipMemcpy(hs.data(), t->s + (size_t)ct0 * nb4 * 64, sw * 2, hipMemcpyDeviceToHost));
  static const int p4[8] = {0, 2, 4, 6, 1, 3, 5, 7};
  static const int p8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
  for (int r = 0; r < n; r++) {
    int ct = r / 16, nn = r % 16;
    for (int b = 0; b < nb; b++) {
      int bq = b / 4, bb = b % 4;
      int q[32];
      for (int g = 0; g < 4; g++) {
        size_t base = (((size_t)ct * nb4 + bq) * 4 + g) * 16 + nn;
        if (bits == 4) {
          uint32_t dw = hw[base * 4 + bb];
          for (int i = 0; i < 8; i++) q[8 * g + p4[i]] = (dw >> (4 * i)) & 15;
        } else {
          uint32_t d0 = hw[(base * 4 + bb) * 2], d1 = hw[(base * 4 + bb) * 2 + 1];
          for (int i = 0; i < 4; i++) {
            q[8 * g + p8[i]] = (int8_t)((d0 >> (8 * i)) & 0xFF);
            q[8 * g + p8[4 + i]] = (int8_t)((d1 >> (8 * i)) & 0xFF);
          }
        }
      }
      if (wq) {
        if (bits == 4) {
          uint8_t* o = (uint8_t*)wq + ((size_t)r * nb + b) * 16;
          for (int j = 0; j < 16; j++) o[j] = (uint8_t)(q[2 * j] | (q[2 * j + 1] << 4));
        } else {
          int8_t* o = (int8_t*)wq + ((size_t)r * nb + b) * 32;
          for (int i = 0; i < 32; i++) o[i] = (int8_t)q[i];
        }
      }
      if (ws) ws[(size_t)r * nb + b] = hs[((((size_t)ct * nb4 + bq) * 4 + (nn >> 2)) * 4 + bb) * 4 + (nn & 3)];
    }
  }
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// page pool
// ---------------------------------------------------------------------------
extern "C" int rstr_pool_open(rstr_model* m, int32_t page_size, int32_t physical_pages, rstr_pool** out) {
  if (!m) return fail(nullptr, RSTR_E_INVALID, "null model");
  rstr_session* s = m->s;
  if (!out) return fail(s, RSTR_E_INVALID, "null output pointer");
  *out = nullptr;
  if (page_size <= 0 || physical_pages <= 0)
    return fail(s, RSTR_E_INVALID, "Page-pool extent must be a positive integer");
  if (page_size % 4) return fail(s, RSTR_E_INVALID, "page size must be a multiple of 4");
  HIPCHK(s, hipSetDevice(s->device));
  auto p = std::make_unique<rstr_pool>();
  p->m = m;
  p->page_size = page_size;
  p->physical_pages = physical_pages;
  p->page_elems = (int64_t)page_size * m->d.n_kv * m->d.head_dim;
  int L = m->d.n_layers;
  size_t slab_elems = (size_t)physical_pages * (size_t)p->page_elems;
  auto cleanup = [&]() {
    for (auto* q : p->slabs) hipFree(q);
    if (p->d_slabs) hipFree(p->d_slabs);
    if (p->d_pairs) hipFree(p->d_pairs);
    if (p->h_pairs) hipHostFree(p->h_pairs);
  };
  for (int i = 0; i < 2 * L; i++) {
    uint16_t* q = nullptr;
    hipError_t e = hipMalloc(&q, slab_elems * 2);
    if (e != hipSuccess) {
      cleanup();
      return fail(s, RSTR_E_OOM, "page pool slab allocation failed");
    }
    p->slabs.push_back(q);
    if (hipMemsetAsync(q, 0, slab_elems * 2, s->stream) != hipSuccess) {
      cleanup();
      return fail(s, RSTR_E_HIP, "page pool clear failed");
    }
  }
  if (dmalloc(&p->d_slabs, 2 * L) != hipSuccess || dmalloc(&p->d_pairs, 2) != hipSuccess ||
      hipHostMalloc((void**)&p->h_pairs, 2 * sizeof(int32_t)) != hipSuccess) {
    cleanup();
    return fail(s, RSTR_E_OOM, "page pool tables");
  }
  if (hipMemcpy(p->d_slabs, p->slabs.data(), sizeof(uint16_t*) * 2 * L, hipMemcpyHostToDevice) !=
          hipSuccess ||
      hipStreamSynchronize(s->stream) != hipSuccess) {
    cleanup();
    return fail(s, RSTR_E_HIP, "page pool setup");
  }
  *out = p.release();
  return RSTR_OK;
}

extern "C" int rstr_pool_close(rstr_pool* p) {
  if (!p) return RSTR_OK;
  if (p->open_transfers > 0) return fail(p->m->s, RSTR_E_STATE, "pool has chunk transfers in flight");
  hipSetDevice(p->m->s->device);
  hipStreamSynchronize(p->m->s->stream);
  for (auto* q : p->slabs) hipFree(q);
  hipFree(p->d_slabs);
  hipFree(p->d_pairs);
  hipHostFree(p->h_pairs);
  if (p->d_fill) hipFree(p->d_fill);
  p->ring.release();
  if (p->tmpl) hipFree(p->tmpl);
  if (p->stage) hipFree(p->stage);
  if (p->d_chunk_pages) hipFree(p->d_chunk_pages);
  for (auto& b : p->pinned) hipHostFree(b.first);
  delete p;
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// durable chunk transfer
// ---------------------------------------------------------------------------
// Keep up to 4 idle pinned buffers per pool (the largest), free the rest.
static void pinned_release(rstr_pool* p, void* host, size_t bytes) {
  p->pinned.emplace_back(host, bytes);
  if (p->pinned.size() > 4) {
    auto smallest = std::min_element(p->pinned.begin(), p->pinned.end(),
                                      [](const auto& a, const auto& b) { return a.second < b.second; });
    hipHostFree(smallest->first);
    p->pinned.erase(smallest);
  }
}

static int chunk_submit(rstr_pool* p, const int32_t* pages, int32_t n_pages, int32_t start, int32_t count,
                        int mode, const void* src, uint16_t* dst, rstr_transfer** out) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  if (!out) return fail(s, RSTR_E_INVALID, "null output pointer");
  *out = nullptr;
  if (!pages || n_pages <= 0) return fail(s, RSTR_E_INVALID, "empty page list");
  if (start < 0 || count <= 0 || (int64_t)start + count > (int64_t)n_pages * p->page_size)
    return fail(s, RSTR_E_INVALID, "Chunk range is outside the resident continuation");
  const int first = start / p->page_size, last = (start + count - 1) / p->page_size;
  for (int i = first; i <= last; i++)
    if (pages[i] < 0 || pages[i] >= p->physical_pages) return fail(s, RSTR_E_INVALID, "page id out of range");
  if ((mode == 0 && !dst) || (mode != 0 && !src)) return fail(s, RSTR_E_INVALID, "null payload");
  const auto& md = p->m->d;
  const int L = md.n_layers, ept = md.n_kv * md.head_dim;
  const size_t elems = (size_t)2 * L * count * ept;
  const size_t pbytes = elems * (mode == 2 ? 4 : 2);
  HIPCHK(s, hipSetDevice(s->device));
  // grow the pool-owned staging (the stream drains first: earlier transfers use it)
  if (p->stage_bytes < pbytes || p->chunk_pages_cap < n_pages) {
    HIPCHK(s, hipStreamSynchronize(s->stream));
    if (p->stage_bytes < pbytes) {
      if (p->stage) hipFree(p->stage);
      p->stage = nullptr;
      p->stage_bytes = 0;
      if (hipMalloc(&p->stage, pbytes) != hipSuccess) return fail(s, RSTR_E_OOM, "chunk staging allocation failed");
      p->stage_bytes = pbytes;
    }
    if (p->chunk_pages_cap < n_pages) {
      if (p->d_chunk_pages) hipFree(p->d_chunk_pages);
      p->d_chunk_pages = nullptr;
      p->chunk_pages_cap = 0;
      if (dmalloc(&p->d_chunk_pages, (size_t)n_pages) != hipSuccess)
        return fail(s, RSTR_E_OOM, "chunk page list allocation failed");
      p->chunk_pages_cap = n_pages;
    }
  }
  auto t = std::make_unique<rstr_transfer>();
  t->p = p;
  t->direction = mode == 0 ? 1 : 0;
  t->payload_bytes = pbytes;
  t->user_dst = dst;
  const size_t pages_bytes = ((size_t)n_pages * 4 + 255) / 256 * 256;
  const size_t need = pages_bytes + pbytes;
  // smallest idle pinned buffer that fits, else a new one
  int best = -1;
  for (int i = 0; i < (int)p->pinned.size(); i++)
    if (p->pinned[i].second >= need && (best < 0 || p->pinned[i].second < p->pinned[best].second)) best = i;
  if (best >= 0) {
    t->host = p->pinned[best].first;
    t->host_bytes = p->pinned[best].second;
    p->pinned.erase(p->pinned.begin() + best);
  } else {
    if (hipHostMalloc(&t->host, need) != hipSuccess) return fail(s, RSTR_E_OOM, "pinned chunk buffer allocation failed");
    t->host_bytes = need;
  }
  auto cleanup = [&]() {
    if (t->e0) hipEventDestroy(t->e0);
    if (t->e1) hipEventDestroy(t->e1);
    pinned_release(p, t->host, t->host_bytes);
  };
  std::memcpy(t->host, pages, (size_t)n_pages * 4);
  t->host_payload_offset = pages_bytes;
  char* hpay = static_cast<char*>(t->host) + pages_bytes;
  if (mode != 0) std::memcpy(hpay, src, pbytes);
  hipError_t e = hipEventCreate(&t->e0);
  if (e == hipSuccess) e = hipEventCreate(&t->e1);
  if (e == hipSuccess) e = hipEventRecord(t->e0, s->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(p->d_chunk_pages, t->host, (size_t)n_pages * 4, hipMemcpyHostToDevice, s->stream);
  if (e == hipSuccess && mode != 0) e = hipMemcpyAsync(p->stage, hpay, pbytes, hipMemcpyHostToDevice, s->stream);
  if (e == hipSuccess)
    e = launch_chunk_move(s->stream, mode, p->d_slabs, 2 * L, p->d_chunk_pages, start, count, p->page_size, ept,
                          p->stage);
  if (e == hipSuccess && mode == 0) e = hipMemcpyAsync(hpay, p->stage, pbytes, hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess) e = hipEventRecord(t->e1, s->stream);
  if (e != hipSuccess) {
    hipStreamSynchronize(s->stream);
    cleanup();
    return fail(s, RSTR_E_HIP, std::string("chunk transfer: ") + hipGetErrorString(e));
  }
  p->open_transfers++;
  *out = t.release();
  return RSTR_OK;
}

extern "C" int rstr_chunk_bench(rstr_pool* p, const int32_t* pages, int32_t n_pages, int32_t start,
                                int32_t token_count, int32_t mode, int32_t iters, float* kernel_ms) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  if ((mode != 0 && mode != 1) || iters <= 0 || !kernel_ms) return fail(s, RSTR_E_INVALID, "invalid bench request");
  // a gather submission sets up staging, page list and validation
  rstr_transfer* t = nullptr;
  std::vector<uint16_t> sink;
  if (token_count > 0 && n_pages > 0)
    sink.resize((size_t)2 * p->m->d.n_layers * token_count * p->m->d.n_kv * p->m->d.head_dim);
  int rc = chunk_submit(p, pages, n_pages, start, token_count, 0, nullptr, sink.data(), &t);
  if (rc) return rc;
  if ((rc = rstr_transfer_complete(t, nullptr))) return rc;
  const int L = p->m->d.n_layers, ept = p->m->d.n_kv * p->m->d.head_dim;
  hipEvent_t a, b;
  HIPCHK(s, hipEventCreate(&a));
  HIPCHK(s, hipEventCreate(&b));
  hipError_t e = hipEventRecord(a, s->stream);
  for (int i = 0; i < iters && e == hipSuccess; i++)
    e = launch_chunk_move(s->stream, mode, p->d_slabs, 2 * L, p->d_chunk_pages, start, token_count, p->page_size,
                          ept, p->stage);
  if (e == hipSuccess) e = hipEventRecord(b, s->stream);
  if (e == hipSuccess) e = hipEventSynchronize(b);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
  hipEventDestroy(a);
  hipEventDestroy(b);
  HIPCHK(s, e);
  *kernel_ms = ms / iters;
  return RSTR_OK;
}

extern "C" int rstr_chunk_export_submit(rstr_pool* p, const int32_t* pages, int32_t n_pages, int32_t start,
                                        int32_t token_count, uint16_t* payload, rstr_transfer** out) {
  return chunk_submit(p, pages, n_pages, start, token_count, 0, nullptr, payload, out);
}

extern "C" int rstr_chunk_restore_submit(rstr_pool* p, const int32_t* pages, int32_t n_pages, int32_t start,
                                         int32_t token_count, const void* payload, int32_t payload_dtype,
                                         rstr_transfer** out) {
  if (p && payload_dtype != 0 && payload_dtype != 1)
    return fail(p->m->s, RSTR_E_INVALID, "Payload dtype and representation cannot be restored to FP16");
  return chunk_submit(p, pages, n_pages, start, token_count, payload_dtype == 1 ? 2 : 1, payload, nullptr, out);
}

extern "C" int rstr_transfer_done(rstr_transfer* t) {
  if (!t) return fail(nullptr, RSTR_E_INVALID, "null transfer");
  hipError_t e = hipEventQuery(t->e1);
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  return fail(t->p->m->s, RSTR_E_HIP, std::string("transfer query: ") + hipGetErrorString(e));
}

extern "C" int rstr_transfer_complete(rstr_transfer* t, rstr_transfer_stats* stats) {
  if (!t) return fail(nullptr, RSTR_E_INVALID, "null transfer");
  std::unique_ptr<rstr_transfer> own(t);
  rstr_pool* p = t->p;
  rstr_session* s = p->m->s;
  p->open_transfers--;
  hipError_t e = hipEventSynchronize(t->e1);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, t->e0, t->e1);
  if (e == hipSuccess && t->direction == 1) {
    // the payload follows the 256-byte aligned page list in the pinned buffer
    const size_t off = t->host_payload_offset;
    std::memcpy(t->user_dst, static_cast<char*>(t->host) + off, t->payload_bytes);
  }
  hipEventDestroy(t->e0);
  hipEventDestroy(t->e1);
  if (e == hipSuccess) pinned_release(p, t->host, t->host_bytes);
  else hipHostFree(t->host);
  if (e != hipSuccess) return fail(s, RSTR_E_HIP, std::string("transfer completion: ") + hipGetErrorString(e));
  if (stats) {
    stats->bytes = (int64_t)t->payload_bytes;
    stats->device_ms = ms;
    stats->direction = t->direction;
  }
  return RSTR_OK;
}

extern "C" int rstr_pool_copy_page(rstr_pool* p, int32_t src, int32_t dst) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  if (src < 0 || dst < 0 || src >= p->physical_pages || dst >= p->physical_pages)
    return fail(s, RSTR_E_INVALID, "Page view does not name a pool page");
  if (src == dst) return RSTR_OK;
  HIPCHK(s, hipSetDevice(s->device));
  // queued in stream order (after every step submitted before it), not waited for
  int32_t* h = nullptr;
  int slot = 0;
  const int32_t pair[2] = {src, dst};
  HIPCHK(s, p->ring.stage(pair, 2, nullptr, 0, &h, &slot));
  HIPCHK(s, hipMemcpyAsync(p->d_pairs, h, 2 * sizeof(int32_t), hipMemcpyHostToDevice, s->stream));
  HIPCHK(s, p->ring.queued(slot, s->stream));
  HIPCHK(s, launch_copy_pages(s->stream, p->d_slabs, 2 * p->m->d.n_layers, p->page_elems, p->d_pairs, 1));
  return RSTR_OK;
}

static int slab_index(rstr_pool* p, int32_t slab, int32_t layer) {
  if (slab < 0 || slab > 1 || layer < 0 || layer >= p->m->d.n_layers) return -1;
  return slab * p->m->d.n_layers + layer;
}

extern "C" int rstr_pool_upload(rstr_pool* p, int32_t slab, int32_t layer, int64_t dst_element,
                                const uint16_t* src, int64_t elements) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  int si = slab_index(p, slab, layer);
  int64_t cap = (int64_t)p->physical_pages * p->page_elems;
  if (si < 0 || dst_element < 0 || elements < 0 || dst_element + elements > cap || (!src && elements))
    return fail(s, RSTR_E_INVALID, "pool upload range is outside the slab");
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  HIPCHK(s, hipMemcpy(p->slabs[si] + dst_element, src, (size_t)elements * 2, hipMemcpyHostToDevice));
  return RSTR_OK;
}

extern "C" int rstr_pool_download(rstr_pool* p, int32_t slab, int32_t layer, int64_t src_element,
                                  uint16_t* dst, int64_t elements) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  int si = slab_index(p, slab, layer);
  int64_t cap = (int64_t)p->physical_pages * p->page_elems;
  if (si < 0 || src_element < 0 || elements < 0 || src_element + elements > cap || (!dst && elements))
    return fail(s, RSTR_E_INVALID, "pool download range is outside the slab");
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  HIPCHK(s, hipMemcpy(dst, p->slabs[si] + src_element, (size_t)elements * 2, hipMemcpyDeviceToHost));
  return RSTR_OK;
}

extern "C" int rstr_pool_fill_synthetic(rstr_pool* p, const int32_t* pages, int32_t n, uint64_t seed) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  if (n < 0 || (n && !pages)) return fail(s, RSTR_E_INVALID, "invalid page list");
  for (int32_t i = 0; i < n; i++)
    if (pages[i] < 0 || pages[i] >= p->physical_pages) return fail(s, RSTR_E_INVALID, "page out of range");
  if (n == 0) return RSTR_OK;
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, ensure_templates(p, seed));
  if (n > p->fill_cap) {  // grows rarely; freeing waits for the device
    HIPCHK(s, hipStreamSynchronize(s->stream));
    if (p->d_fill) hipFree(p->d_fill);
    p->d_fill = nullptr;
    p->fill_cap = 0;
    const int cap = std::max(n, 1024);
    HIPCHK(s, dmalloc(&p->d_fill, cap));
    p->fill_cap = cap;
  }
  // queued in stream order (after every step submitted before it), not waited for
  int32_t* h = nullptr;
  int slot = 0;
  HIPCHK(s, p->ring.stage(pages, n, nullptr, 0, &h, &slot));
  HIPCHK(s, hipMemcpyAsync(p->d_fill, h, sizeof(int32_t) * n, hipMemcpyHostToDevice, s->stream));
  HIPCHK(s, p->ring.queued(slot, s->stream));
  HIPCHK(s, launch_fill_synthetic(s->stream, p->d_slabs, p->m->d.n_layers, p->page_elems, p->tmpl, p->d_fill, n,
                                  seed));
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// paged decoder
// ---------------------------------------------------------------------------
static void decoder_free(rstr_decoder* d) {
  if (!d) return;
  hipSetDevice(d->m->s->device);
  if (d->graph) hipGraphExecDestroy(d->graph);
  for (void* q : {(void*)d->r0, (void*)d->xmid, (void*)d->o, (void*)d->yqkv, (void*)d->qr, (void*)d->gu,
                  (void*)d->logits, (void*)d->part, (void*)d->rope_cos, (void*)d->rope_sin,
                  (void*)d->act.q, (void*)d->act.s, (void*)d->act_ff.q, (void*)d->act_ff.s,
                  (void*)d->desc, (void*)d->lane_tab,
                  (void*)d->tokbuf, (void*)d->amax_cand, (void*)d->d_lanes, (void*)d->d_tokens,
                  (void*)d->sched_desc, (void*)d->sched_pages, (void*)d->sched_tok})
    if (q) hipFree(q);
  if (d->h_desc) hipHostFree(d->h_desc);
  if (d->h_tok) hipHostFree(d->h_tok);
  for (hipEvent_t ev : d->ev_step)
    if (ev) hipEventDestroy(ev);
  for (int i = 0; i < 2; i++) {
    if (d->h_desc_q[i]) hipHostFree(d->h_desc_q[i]);
    if (d->h_tok_q[i]) hipHostFree(d->h_tok_q[i]);
    if (d->ev_q[i]) hipEventDestroy(d->ev_q[i]);
  }
  d->ring.release();
  delete d;
}

static int decoder_open(rstr_model* m, rstr_pool* p, int32_t batch, int32_t pps, int32_t maxpos,
                        int32_t split, bool head_tail, rstr_decoder** out) {
  if (!m || !p) return fail(nullptr, RSTR_E_INVALID, "null model or pool");
  rstr_session* s = m->s;
  if (!out) return fail(s, RSTR_E_INVALID, "null output pointer");
  *out = nullptr;
  if (p->m != m) return fail(s, RSTR_E_INVALID, "pool belongs to another model");
  if (batch <= 0 || pps <= 0 || maxpos <= 0)
    return fail(s, RSTR_E_INVALID, "Paged decoder capacity must be a positive integer");
  if (split <= 0 || split % 4 || split > 4096)
    return fail(s, RSTR_E_INVALID, "attention split must be a positive multiple of 4 up to 4096");
  if (batch > 4096) return fail(s, RSTR_E_INVALID, "batch too large");
  HIPCHK(s, hipSetDevice(s->device));
  const auto& md = m->d;
  auto d = new rstr_decoder();
  d->m = m;
  d->p = p;
  d->B = batch;
  d->pps = pps;
  d->maxpos = maxpos;
  d->split = split;
  d->head_tail = head_tail;
  d->mpad = (batch + 15) / 16 * 16;
  d->qd = md.n_q * md.head_dim;
  d->kvr = md.n_kv * md.head_dim;
  d->nqkv = d->qd + 2 * d->kvr;
  d->kmax = std::max(md.d_model, std::max(d->qd, md.d_ff));
  d->s_qkv = qgemm_splits(d->nqkv, d->mpad, md.weight_bits);
  d->s_o = qgemm_splits(md.d_model, d->mpad, md.weight_bits);
  d->s_gu = qgemm_splits(2 * md.d_ff, d->mpad, md.weight_bits);
  d->s_down = qgemm_splits(md.d_model, d->mpad, md.weight_bits);
  const int s_d = std::max(d->s_o, d->s_down);
  int64_t max_pos_tokens = std::min<int64_t>((int64_t)pps * p->page_size, (int64_t)maxpos + 1);
  int64_t splits = (max_pos_tokens + split - 1) / split + 1;
  d->max_items = (int)std::min<int64_t>((int64_t)batch * md.n_kv * splits, INT32_MAX / 4);
  int G = md.n_q / md.n_kv;
  d->off_slots = 0;
  d->off_rows = batch;
  d->off_pos = d->off_rows + batch + 1;
  d->off_len = d->off_pos + batch;
  d->off_start = d->off_len + batch;
  d->off_pt = d->off_start + batch;
  d->desc_words = d->off_pt + (int64_t)batch * pps;
  int half = md.head_dim / 2;
  hipError_t e = hipSuccess;
  auto A = [&](hipError_t x) { if (e == hipSuccess) e = x; };
  A(dmalloc(&d->r0, (size_t)d->mpad * md.d_model));
  A(dmalloc(&d->xmid, (size_t)d->mpad * md.d_model));
  A(dmalloc(&d->o, (size_t)s_d * batch * md.d_model));
  A(dmalloc(&d->yqkv, (size_t)d->s_qkv * batch * d->nqkv));
  A(dmalloc(&d->qr, (size_t)batch * d->qd));
  d->fuse_act = qgemm_act_fused(md.d_ff, d->mpad);
  if (!d->fuse_act) A(dmalloc(&d->gu, (size_t)d->s_gu * batch * 2 * md.d_ff));
  if (head_tail) A(dmalloc(&d->logits, (size_t)batch * md.vocab));
  A(dmalloc(&d->part, (size_t)d->max_items * G * attn_part_floats(md.head_dim)));
  A(dmalloc(&d->rope_cos, (size_t)2 * maxpos * half));
  A(dmalloc(&d->rope_sin, (size_t)2 * maxpos * half));
  A(dmalloc(&d->act.q, (size_t)d->mpad * d->kmax));
  A(dmalloc(&d->act.s, (size_t)d->mpad * (d->kmax / 32)));
  if (d->fuse_act) {
    A(dmalloc(&d->act_ff.q, (size_t)d->mpad * md.d_ff));
    A(dmalloc(&d->act_ff.s, (size_t)d->mpad * (md.d_ff / 32)));
  }
  A(dmalloc(&d->desc, (size_t)d->desc_words));
  d->tabw = attn_tab_words(AttnGeom{batch, md.n_q, md.n_kv, md.head_dim, p->page_size, pps, split, 0,
                                     md.attn_scale}, d->max_items);
  if (d->tabw == 0 && e == hipSuccess) e = hipErrorInvalidValue;
  d->fuse_qkv = head_tail && d->tabw && attn_fuses_qkv(AttnGeom{batch, md.n_q, md.n_kv, md.head_dim, p->page_size, pps,
                                                                split, 0, md.attn_scale}, d->max_items);
  d->attn_direct = head_tail && d->tabw && maxpos <= split &&
                   attn_direct_out(AttnGeom{batch, md.n_q, md.n_kv, md.head_dim, p->page_size, pps, split, 0,
                                            md.attn_scale}, d->max_items);
  A(dmalloc(&d->lane_tab, 2 * d->tabw));
  A(dmalloc(&d->tokbuf, (size_t)batch));
  A(dmalloc(&d->amax_cand, (size_t)2 * batch * argmax_segments(batch, md.vocab)));
  A(dmalloc(&d->d_lanes, (size_t)batch));
  A(dmalloc(&d->d_tokens, (size_t)batch));
  if (e == hipSuccess) e = hipHostMalloc((void**)&d->h_desc, sizeof(int32_t) * d->desc_words);
  if (e == hipSuccess) e = hipHostMalloc((void**)&d->h_tok, sizeof(int32_t) * batch);
  for (hipEvent_t& ev : d->ev_step)
    if (e == hipSuccess) e = hipEventCreate(&ev);
  for (int i = 0; i < 2; i++) {
    if (e == hipSuccess) e = hipHostMalloc((void**)&d->h_desc_q[i], sizeof(int32_t) * d->desc_words);
    if (e == hipSuccess) e = hipHostMalloc((void**)&d->h_tok_q[i], sizeof(int32_t) * batch);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&d->ev_q[i], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    decoder_free(d);
    return fail(s, RSTR_E_OOM, std::string("decoder allocation: ") + hipGetErrorString(e));
  }
  d->act.mpad = d->mpad;
  d->act_ff.mpad = d->mpad;
  // RoPE tables: table 0 = global theta, table 1 = local theta; double angles.
  {
    std::vector<float> c((size_t)2 * maxpos * half), sn((size_t)2 * maxpos * half);
    for (int t = 0; t < 2; t++) {
      double theta = t == 0 ? md.rope_global : md.rope_local;
      for (int ps = 0; ps < maxpos; ps++)
        for (int i = 0; i < half; i++) {
          double inv = std::pow(theta, -(2.0 * (double)i) / (double)md.head_dim);
          double ang = (double)ps * inv;
          size_t k = ((size_t)t * maxpos + ps) * half + i;
          c[k] = (float)std::cos(ang);
          sn[k] = (float)std::sin(ang);
        }
    }
    A(hipMemcpy(d->rope_cos, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    A(hipMemcpy(d->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  }
  A(hipMemset(d->r0, 0, sizeof(float) * d->mpad * md.d_model));
  A(hipMemset(d->act.q, 0, sizeof(_Float16) * d->mpad * d->kmax));
  A(hipMemset(d->act.s, 0, sizeof(float) * d->mpad * (d->kmax / 32)));
  if (d->fuse_act) {
    A(hipMemset(d->act_ff.q, 0, sizeof(_Float16) * d->mpad * md.d_ff));
    A(hipMemset(d->act_ff.s, 0, sizeof(float) * d->mpad * (md.d_ff / 32)));
  }
  A(hipDeviceSynchronize());
  if (e != hipSuccess) {
    decoder_free(d);
    return fail(s, RSTR_E_HIP, std::string("decoder setup: ") + hipGetErrorString(e));
  }
  *out = d;
  return RSTR_OK;
}

extern "C" int rstr_decoder_open(rstr_model* m, rstr_pool* p, int32_t batch, int32_t pps, int32_t maxpos,
                                 int32_t split, rstr_decoder** out) {
  return decoder_open(m, p, batch, pps, maxpos, split, true, out);
}

extern "C" int rstr_prefill_open(rstr_model* m, rstr_pool* p, int32_t rows, int32_t pps, int32_t maxpos,
                                 int32_t split, rstr_decoder** out) {
  if (m && rows > maxpos) return fail(m->s, RSTR_E_INVALID, "prefill-T must fit in maxpos");
  return decoder_open(m, p, rows, pps, maxpos, split, false, out);
}

extern "C" int rstr_decoder_close(rstr_decoder* d) {
  if (!d) return RSTR_OK;
  hipSetDevice(d->m->s->device);
  hipStreamSynchronize(d->m->s->stream);
  decoder_free(d);
  return RSTR_OK;
}

extern "C" int rstr_decoder_set_graph(rstr_decoder* d, int32_t enabled) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  d->use_graph = enabled != 0;
  return RSTR_OK;
}

static int check_lanes(rstr_decoder* d, int32_t n, const int32_t* lanes) {
  rstr_session* s = d->m->s;
  if (n < 0 || n > d->B || (n && !lanes)) return fail(s, RSTR_E_INVALID, "invalid lane list");
  std::vector<char> seen(d->B, 0);
  for (int32_t i = 0; i < n; i++) {
    if (lanes[i] < 0 || lanes[i] >= d->B || seen[lanes[i]])
      return fail(s, RSTR_E_INVALID, "Resident token lanes are invalid for the bound decoder");
    seen[lanes[i]] = 1;
  }
  return RSTR_OK;
}

extern "C" int rstr_prime_lanes(rstr_decoder* d, int32_t n, const int32_t* lanes, const int32_t* tokens) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  int rc = check_lanes(d, n, lanes);
  if (rc) return rc;
  for (int32_t i = 0; i < n; i++)
    if (!tokens || tokens[i] < 0 || tokens[i] >= d->m->d.vocab)
      return fail(s, RSTR_E_INVALID, "token id out of range");
  if (n == 0) return RSTR_OK;
  HIPCHK(s, hipSetDevice(s->device));
  // queued in stream order (after every step submitted before it), not waited for
  int32_t* h = nullptr;
  int slot = 0;
  HIPCHK(s, d->ring.stage(lanes, n, tokens, n, &h, &slot));
  HIPCHK(s, hipMemcpyAsync(d->d_lanes, h, sizeof(int32_t) * n, hipMemcpyHostToDevice, s->stream));
  HIPCHK(s, hipMemcpyAsync(d->d_tokens, h + n, sizeof(int32_t) * n, hipMemcpyHostToDevice, s->stream));
  HIPCHK(s, d->ring.queued(slot, s->stream));
  HIPCHK(s, launch_gather_rows(s->stream, d->m->emb, d->m->d.d_model, d->d_lanes, d->d_tokens, n, d->r0));
  return RSTR_OK;
}

extern "C" int rstr_prime_rows(rstr_decoder* d, int32_t n, const int32_t* lanes, const float* rows) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  int rc = check_lanes(d, n, lanes);
  if (rc) return rc;
  if (n && !rows) return fail(s, RSTR_E_INVALID, "null rows");
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  int dm = d->m->d.d_model;
  for (int32_t i = 0; i < n; i++)
    HIPCHK(s, hipMemcpy(d->r0 + (size_t)lanes[i] * dm, rows + (size_t)i * dm, sizeof(float) * dm,
                        hipMemcpyHostToDevice));
  return RSTR_OK;
}

extern "C" int rstr_decoder_read_rows(rstr_decoder* d, float* out) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  HIPCHK(s, hipMemcpy(out, d->r0, sizeof(float) * d->B * d->m->d.d_model, hipMemcpyDeviceToHost));
  return RSTR_OK;
}

extern "C" int rstr_decode_logits(rstr_decoder* d, float* out) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  if (!d->has_logits) return fail(s, RSTR_E_STATE, "no step has run");
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  HIPCHK(s, hipMemcpy(out, d->logits, sizeof(float) * d->B * d->m->d.vocab, hipMemcpyDeviceToHost));
  return RSTR_OK;
}

// Validation of one step's descriptors (the checks Raster's
// attention/validate-routing! and validate-query-values! make, plus the
// decode invariant that the appended row is the route's last visible token).
// True when no lane's visible range holds another lane's append slot, i.e.
// each lane's new K/V row is read only by that lane in this step (what the
// page pool's copy-on-write guarantees for decode; bulk-prefill tiles are the
// opposite case).  Run on validated descriptors.
static bool appends_private(rstr_decoder* d, const int32_t* slots, const int32_t* pt, const int32_t* len) {
  const int ps = d->p->page_size;
  auto& mk = d->mark;
  if ((int64_t)mk.size() != (int64_t)d->p->physical_pages) mk.assign(d->p->physical_pages, -1);
  bool ok = true;
  for (int b = 0; b < d->B; b++) {
    if (slots[b] < 0) continue;
    const int32_t P = slots[b] / ps;
    if (mk[P] != -1) ok = false;  // two appends in one page
    mk[P] = b;
  }
  for (int c = 0; ok && c < d->B; c++) {
    const int32_t L = len[c];
    const int32_t* row = pt + (int64_t)c * d->pps;
    for (int32_t i = 0; i < (L + ps - 1) / ps; i++) {
      const int32_t b = mk[row[i]];
      if (b >= 0 && b != c && (int64_t)i * ps + slots[b] % ps < L) {
        ok = false;
        break;
      }
    }
  }
  for (int b = 0; b < d->B; b++)
    if (slots[b] >= 0) mk[slots[b] / ps] = -1;
  return ok;
}

static int validate_step(rstr_decoder* d, const int32_t* slots, const int32_t* rows, const int32_t* pos,
                         const int32_t* pt, const int32_t* len, const int32_t* start, bool* fused = nullptr) {
  if (fused) *fused = false;
  rstr_session* s = d->m->s;
  if (!slots || !rows || !pos || !pt || !len || !start) return fail(s, RSTR_E_INVALID, "null descriptor");
  int ps = d->p->page_size;
  int64_t slot_limit = (int64_t)d->p->physical_pages * ps;
  for (int b = 0; b <= d->B; b++)
    if (rows[b] != b) return fail(s, RSTR_E_INVALID, "row offsets must be 0..batch for decode");
  for (int b = 0; b < d->B; b++) {
    int32_t L = len[b];
    if (L < 0 || (int64_t)L > (int64_t)d->pps * ps) return fail(s, RSTR_E_INVALID, "lane length out of range");
    if (slots[b] < -1 || slots[b] >= slot_limit) return fail(s, RSTR_E_INVALID, "append slot out of range");
    // every row (idle ones too) is rotated at its position: the RoPE tables
    // hold maxpos rows
    if (pos[b] < 0 || pos[b] >= d->maxpos) return fail(s, RSTR_E_INVALID, "query position outside the decoder's maxpos");
    // a route starts at a non-negative absolute position (page_pool.clj:647)
    if (start[b] < 0) return fail(s, RSTR_E_INVALID, "Resident route identity and extents are invalid");
    if (L == 0) {
      if (slots[b] != -1) return fail(s, RSTR_E_INVALID, "inactive lane has an append slot");
      continue;
    }
    if ((int64_t)pos[b] != (int64_t)start[b] + L - 1)
      return fail(s, RSTR_E_INVALID, "query position must be the route's last visible token");
    int32_t np = (L + ps - 1) / ps;
    const int32_t* row = pt + (int64_t)b * d->pps;
    for (int32_t i = 0; i < np; i++)
      if (row[i] < 0 || row[i] >= d->p->physical_pages)
        return fail(s, RSTR_E_INVALID, "page table entry out of range");
    if (slots[b] >= 0) {
      int32_t t = L - 1;
      int64_t want = (int64_t)row[t / ps] * ps + t % ps;
      if (want != slots[b]) return fail(s, RSTR_E_INVALID, "append slot is not the route's last token");
    }
  }
  if (fused) *fused = d->fuse_qkv && appends_private(d, slots, pt, len);
  return RSTR_OK;
}

static void pack_desc(rstr_decoder* d, int32_t* dst, const int32_t* slots, const int32_t* rows,
                      const int32_t* pos, const int32_t* pt, const int32_t* len, const int32_t* start) {
  std::memcpy(dst + d->off_slots, slots, sizeof(int32_t) * d->B);
  std::memcpy(dst + d->off_rows, rows, sizeof(int32_t) * (d->B + 1));
  std::memcpy(dst + d->off_pos, pos, sizeof(int32_t) * d->B);
  std::memcpy(dst + d->off_len, len, sizeof(int32_t) * d->B);
  std::memcpy(dst + d->off_start, start, sizeof(int32_t) * d->B);
  std::memcpy(dst + d->off_pt, pt, sizeof(int32_t) * (size_t)d->B * d->pps);
}

// Per-kernel-class timing (eager profiling only).
struct Prof {
  std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> marks;
  std::vector<hipEvent_t> pool;
  size_t used = 0;
  hipEvent_t get() {
    if (used == pool.size()) {
      hipEvent_t e;
      hipEventCreate(&e);
      pool.push_back(e);
    }
    return pool[used++];
  }
  ~Prof() { for (auto e : pool) hipEventDestroy(e); }
};

// Enqueue the whole decode step on `st`; every kernel reads descriptors from
// device memory so the sequence can be captured once and replayed.
static hipError_t enqueue_step(rstr_decoder* d, hipStream_t st, Prof* prof, bool fused) {
  const auto& md = d->m->d;
  const int B = d->B, dm = md.d_model, hd = md.head_dim;
  const float goff = md.gain_offset ? 1.0f : 0.0f;
  const int32_t* slots = d->desc + d->off_slots;
  const int32_t* pos = d->desc + d->off_pos;
  const int32_t* len = d->desc + d->off_len;
  const int32_t* pt = d->desc + d->off_pt;
  const bool has_window = md.sliding_window > 0;
  hipError_t e = hipSuccess;
  auto run = [&](int cls, auto&& fn) {
    if (e != hipSuccess) return;
    hipEvent_t a = nullptr, b = nullptr;
    if (prof) {
      a = prof->get();
      b = prof->get();
      hipEventRecord(a, st);
    }
    e = fn();
    if (prof && e == hipSuccess) {
      hipEventRecord(b, st);
      prof->marks.push_back({cls, {a, b}});
    }
  };
  AttnGeom geo[2];
  for (int w = 0; w < 2; w++) {
    geo[w] = AttnGeom{B, md.n_q, md.n_kv, hd, d->p->page_size, d->pps, d->split,
                      w == 1 ? md.sliding_window : 0, md.attn_scale};
  }
  const size_t tabw = d->tabw;
  run(RSTR_K_ROWS, [&] { return launch_attn_lists(st, geo, has_window ? 2 : 1, len, d->lane_tab, tabw, d->max_items); });
  run(RSTR_K_ROWS, [&] {
    return launch_rms_quant(st, d->r0, d->m->layers[0].attn_norm, goff, md.eps, B, dm, d->act);
  });
  const int L = md.n_layers;
  for (int l = 0; l < L; l++) {
    LayerW& W = d->m->layers[l];
    const bool glob = global_layer(md, l);
    const int ti = (md.rope_dual && !glob) ? 1 : 0;
    const int wi = (has_window && !glob) ? 1 : 0;
    const int half = hd / 2;
    uint16_t* kp = d->p->slabs[l];
    uint16_t* vp = d->p->slabs[L + l];
    const size_t sq = (size_t)B * d->nqkv, sd = (size_t)B * dm, sg = (size_t)B * 2 * md.d_ff;
    run(RSTR_K_QGEMM, [&] { return launch_qgemm(st, W.qkv, d->act, B, d->yqkv, d->nqkv, d->s_qkv, sq); });
    const AttnOut aout{d->act.q, d->act.s, d->act.mpad};
    const float* cos_l = d->rope_cos + (size_t)ti * d->maxpos * half;
    const float* sin_l = d->rope_sin + (size_t)ti * d->maxpos * half;
    if (fused) {
      // qk-norm, RoPE and the K/V append in the few-item attention kernel's prologue
      run(RSTR_K_ATTN_SPLIT, [&] {
        const AttnQkv qk{Slices{d->yqkv, d->s_qkv, sq}, W.q_norm, W.k_norm, goff, md.eps, cos_l, sin_l, pos, slots,
                         len, kp, vp};
        return launch_attn_split_qkv(st, geo[wi], qk, pt, d->lane_tab + wi * tabw, d->part, d->max_items,
                                     d->attn_direct ? &aout : nullptr);
      });
    } else {
      run(RSTR_K_QKV_POST, [&] {
        return launch_qkv_post(st, Slices{d->yqkv, d->s_qkv, sq}, B, md.n_q, md.n_kv, hd, W.q_norm, W.k_norm, goff,
                               md.eps, cos_l, sin_l, pos, slots, d->qr, kp, vp);
      });
      run(RSTR_K_ATTN_SPLIT, [&] {
        return launch_attn_split(st, geo[wi], d->qr, kp, vp, pt, d->lane_tab + wi * tabw, d->part, d->max_items,
                                 d->attn_direct ? &aout : nullptr);
      });
    }
    if (!d->attn_direct)
      run(RSTR_K_ATTN_MERGE, [&] {
        return launch_attn_merge(st, geo[wi], len, d->lane_tab + wi * tabw, d->part, nullptr, &d->act);
      });
    run(RSTR_K_QGEMM, [&] { return launch_qgemm(st, W.o, d->act, B, d->o, dm, d->s_o, sd); });
    run(RSTR_K_ROWS, [&] {
      return launch_post_attn(st, Slices{d->o, d->s_o, sd}, d->r0, d->xmid, W.post_attn_norm, W.ffn_pre_norm, goff, md.eps, B,
                              dm, d->act);
    });
    if (d->fuse_act) {
      // gate/up over all of K per workgroup with act(gate)*up quantised in its epilogue
      run(RSTR_K_QGEMM, [&] { return launch_qgemm_act(st, W.gu, d->act, B, md.d_ff, md.ffn_geglu, d->act_ff); });
      run(RSTR_K_QGEMM, [&] { return launch_qgemm(st, W.down, d->act_ff, B, d->o, dm, d->s_down, sd); });
    } else {
      run(RSTR_K_QGEMM, [&] { return launch_qgemm(st, W.gu, d->act, B, d->gu, 2 * md.d_ff, d->s_gu, sg); });
      // few rows: the down projection computes act(gate)*up while staging its
      // input; shapes it does not serve run the activation launch first
      bool down_done = false;
      run(RSTR_K_QGEMM, [&] {
        const hipError_t r = launch_qgemm_actin(st, W.down, ActIn{d->gu, sg, d->s_gu, md.d_ff, md.ffn_geglu},
                                                d->mpad, B, d->o, dm, d->s_down, sd);
        down_done = r == hipSuccess;
        return r == hipErrorNotSupported ? hipSuccess : r;
      });
      if (!down_done) {
        run(RSTR_K_ROWS, [&] {
          return launch_act_quant(st, Slices{d->gu, d->s_gu, sg}, B, md.d_ff, md.ffn_geglu, d->act);
        });
        run(RSTR_K_QGEMM, [&] { return launch_qgemm(st, W.down, d->act, B, d->o, dm, d->s_down, sd); });
      }
    }
    const float* gnext = (l + 1 < L) ? d->m->layers[l + 1].attn_norm : d->m->final_norm;
    run(RSTR_K_ROWS, [&] {
      return launch_post_ffn(st, Slices{d->o, d->s_down, sd}, d->xmid, d->r0, W.ffn_post_norm, gnext, goff, md.eps, B, dm, d->act);
    });
  }
  if (!d->head_tail) return e;
  run(RSTR_K_HEAD, [&] {
    return launch_qgemm(st, d->m->head, d->act, B, d->logits, md.vocab, 1, (size_t)B * md.vocab);
  });
  run(RSTR_K_TAIL, [&] {
    return launch_argmax_gather(st, d->logits, B, md.vocab, d->m->emb, dm, d->tokbuf, d->r0, d->amax_cand);
  });
  return e;
}

// The step graph is captured in the decoder's own form (fused qkv when
// fuse_qkv); a step that cannot take that form runs eagerly.
static int run_step_device(rstr_decoder* d, bool fused) {
  rstr_session* s = d->m->s;
  if (d->use_graph && fused == d->fuse_qkv) {
    if (!d->graph) {
      hipGraph_t g = nullptr;
      HIPCHK(s, hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
      hipError_t e = enqueue_step(d, s->stream, nullptr, d->fuse_qkv);
      hipError_t e2 = hipStreamEndCapture(s->stream, &g);
      if (e != hipSuccess || e2 != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return fail(s, RSTR_E_HIP, std::string("graph capture: ") +
                                       hipGetErrorString(e != hipSuccess ? e : e2));
      }
      hipError_t e3 = hipGraphInstantiate(&d->graph, g, nullptr, nullptr, 0);
      hipGraphDestroy(g);
      HIPCHK(s, e3);
    }
    HIPCHK(s, hipGraphLaunch(d->graph, s->stream));
  } else {
    HIPCHK(s, enqueue_step(d, s->stream, nullptr, fused));
  }
  d->has_logits = d->head_tail;
  return RSTR_OK;
}

extern "C" int rstr_step_lanes(rstr_decoder* d, const int32_t* slots, const int32_t* row_offsets,
                               const int32_t* positions, const int32_t* page_table, const int32_t* lengths,
                               const int32_t* start_positions, int32_t* tokens_out) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  if (!d->head_tail) return fail(s, RSTR_E_STATE, "a bulk-prefill decoder has no head; use rstr_prefill_range");
  using clk = std::chrono::steady_clock;
  const auto t0 = clk::now();
  bool fused = false;
  int rc = validate_step(d, slots, row_offsets, positions, page_table, lengths, start_positions, &fused);
  if (rc) return rc;
  if (!tokens_out) return fail(s, RSTR_E_INVALID, "null token output");
  const auto t1 = clk::now();
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  const auto t2 = clk::now();
  pack_desc(d, d->h_desc, slots, row_offsets, positions, page_table, lengths, start_positions);
  const auto t3 = clk::now();
  HIPCHK(s, hipMemcpyAsync(d->desc, d->h_desc, sizeof(int32_t) * d->desc_words, hipMemcpyHostToDevice,
                           s->stream));
  HIPCHK(s, hipEventRecord(d->ev_step[0], s->stream));
  if ((rc = run_step_device(d, fused))) return rc;
  HIPCHK(s, hipEventRecord(d->ev_step[1], s->stream));
  HIPCHK(s, hipMemcpyAsync(d->h_tok, d->tokbuf, sizeof(int32_t) * d->B, hipMemcpyDeviceToHost, s->stream));
  const auto t4 = clk::now();
  HIPCHK(s, hipStreamSynchronize(s->stream));
  const auto t5 = clk::now();
  std::memcpy(tokens_out, d->h_tok, sizeof(int32_t) * d->B);
  const auto t6 = clk::now();
  auto ms = [](clk::time_point a, clk::time_point b) { return std::chrono::duration<double, std::milli>(b - a).count(); };
  float dev = 0.0f;
  HIPCHK(s, hipEventElapsedTime(&dev, d->ev_step[0], d->ev_step[1]));
  const double v[RSTR_STEP_TIMING_FIELDS] = {ms(t0, t1), ms(t1, t2), ms(t2, t3), ms(t3, t4), ms(t4, t5), ms(t5, t6),
                                             ms(t0, t6), (double)dev};
  std::memcpy(d->step_ms, v, sizeof v);
  return RSTR_OK;
}


// The same step without waiting for it (no counterpart in the reference,
// whose step-lanes! is synchronous): validation, descriptor packing into one
// of two pinned slots, the descriptor copy, the step graph and the token copy
// are enqueued on the session's stream and the call returns.  At most two
// steps are in flight; rstr_step_lanes_collect returns their tokens in
// submission order.  Calls that synchronise the stream (priming, page copies,
// fills, rstr_step_lanes) run after the submitted steps, in stream order.
extern "C" int rstr_step_lanes_submit(rstr_decoder* d, const int32_t* slots, const int32_t* row_offsets,
                                      const int32_t* positions, const int32_t* page_table,
                                      const int32_t* lengths, const int32_t* start_positions) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  if (!d->head_tail) return fail(s, RSTR_E_STATE, "a bulk-prefill decoder has no head; use rstr_prefill_range");
  if (d->q_n >= 2) return fail(s, RSTR_E_STATE, "two submitted steps are in flight: collect one first");
  bool fused = false;
  int rc = validate_step(d, slots, row_offsets, positions, page_table, lengths, start_positions, &fused);
  if (rc) return rc;
  HIPCHK(s, hipSetDevice(s->device));
  // this slot's previous step was collected, so its staging is free
  const int slot = (d->q_first + d->q_n) % 2;
  pack_desc(d, d->h_desc_q[slot], slots, row_offsets, positions, page_table, lengths, start_positions);
  HIPCHK(s, hipMemcpyAsync(d->desc, d->h_desc_q[slot], sizeof(int32_t) * d->desc_words, hipMemcpyHostToDevice,
                           s->stream));
  if ((rc = run_step_device(d, fused))) return rc;
  HIPCHK(s, hipMemcpyAsync(d->h_tok_q[slot], d->tokbuf, sizeof(int32_t) * d->B, hipMemcpyDeviceToHost, s->stream));
  HIPCHK(s, hipEventRecord(d->ev_q[slot], s->stream));
  d->q_n++;
  return RSTR_OK;
}

extern "C" int rstr_step_lanes_collect(rstr_decoder* d, int32_t* tokens_out) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  if (d->q_n == 0) return fail(s, RSTR_E_STATE, "no submitted step is in flight");
  if (!tokens_out) return fail(s, RSTR_E_INVALID, "null token output");
  const int slot = d->q_first;
  HIPCHK(s, hipEventSynchronize(d->ev_q[slot]));
  std::memcpy(tokens_out, d->h_tok_q[slot], sizeof(int32_t) * d->B);
  d->q_first = (slot + 1) % 2;
  d->q_n--;
  return RSTR_OK;
}

extern "C" int rstr_decoder_step_timing(rstr_decoder* d, double* out, int32_t n) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  if (!out || n < 0) return fail(d->m->s, RSTR_E_INVALID, "null timing output");
  std::memcpy(out, d->step_ms, sizeof(double) * (size_t)std::min<int32_t>(n, RSTR_STEP_TIMING_FIELDS));
  return RSTR_OK;
}

// One complete tile of `rows` prompt tokens of one route: row i is a causal
// lane whose visible range is [start, positions[i]] of the same page-table row,
// so every row's attention and projections follow the decode step's reduction
// order and the K/V written equal token-by-token priming bit for bit.
extern "C" int rstr_prefill_range(rstr_decoder* d, const int32_t* tokens, const int32_t* slots,
                                  const int32_t* positions, const int32_t* page_table, int32_t length,
                                  int32_t start_position) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  if (d->head_tail) return fail(s, RSTR_E_STATE, "Paged decoder has no resident bulk-prefill executable");
  if (!tokens || !slots || !positions || !page_table) return fail(s, RSTR_E_INVALID, "null descriptor");
  const int T = d->B;
  std::vector<int32_t> rows(T + 1), len(T), start(T, start_position), pt((size_t)T * d->pps), lanes(T);
  for (int i = 0; i < T; i++) {
    if (tokens[i] < 0 || tokens[i] >= d->m->d.vocab) return fail(s, RSTR_E_INVALID, "token id out of range");
    int64_t L = (int64_t)positions[i] - start_position + 1;
    if (L < 1 || L > length) return fail(s, RSTR_E_INVALID, "prefill row position outside the route");
    len[i] = (int32_t)L;
    rows[i] = i;
    lanes[i] = i;
    std::memcpy(pt.data() + (size_t)i * d->pps, page_table, sizeof(int32_t) * d->pps);
  }
  rows[T] = T;
  int rc = validate_step(d, slots, rows.data(), positions, pt.data(), len.data(), start.data());
  if (rc) return rc;
  for (int i = 0; i < T; i++)
    if (slots[i] < 0) return fail(s, RSTR_E_INVALID, "every prefill row appends its K/V");
  if ((rc = rstr_prime_lanes(d, T, lanes.data(), tokens))) return rc;
  pack_desc(d, d->h_desc, slots, rows.data(), positions, pt.data(), len.data(), start.data());
  HIPCHK(s, hipMemcpyAsync(d->desc, d->h_desc, sizeof(int32_t) * d->desc_words, hipMemcpyHostToDevice,
                           s->stream));
  if ((rc = run_step_device(d, false))) return rc;
  HIPCHK(s, hipStreamSynchronize(s->stream));
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// schedules (measurement)
// ---------------------------------------------------------------------------
extern "C" int rstr_schedule_upload(rstr_decoder* d, const rstr_staged_step* steps, int32_t n) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  if (!d->head_tail) return fail(s, RSTR_E_STATE, "schedules replay decode steps, not prefill tiles");
  if (n <= 0 || !steps) return fail(s, RSTR_E_INVALID, "empty schedule");
  int64_t words = 0, pages = 0;
  uint64_t fill_seed = 0;
  bool fill_seed_set = false;
  std::unique_ptr<bool[]> fused_steps(new bool[n]());
  for (int32_t i = 0; i < n; i++) {
    const auto& t = steps[i];
    int rc = validate_step(d, t.slots, t.row_offsets, t.positions, t.page_table, t.lengths,
                           t.start_positions, &fused_steps[i]);
    if (rc) return rc;
    if (t.n_fill < 0 || t.n_cow < 0 || (t.n_fill && !t.fill_pages) || (t.n_cow && !t.cow_pairs))
      return fail(s, RSTR_E_INVALID, "invalid staged fill or copy list");
    if (t.n_prime < 0 || t.n_prime > d->B || (t.n_prime && (!t.prime_lanes || !t.prime_tokens)))
      return fail(s, RSTR_E_INVALID, "invalid staged prime list");
    if (int rc2 = check_lanes(d, t.n_prime, t.prime_lanes)) return rc2;
    for (int32_t j = 0; j < t.n_prime; j++)
      if (t.prime_tokens[j] < 0 || t.prime_tokens[j] >= d->m->d.vocab)
        return fail(s, RSTR_E_INVALID, "staged prime token out of range");
    if (t.n_fill && fill_seed_set && t.fill_seed != fill_seed)
      return fail(s, RSTR_E_INVALID, "one schedule uses one synthetic fill seed");
    if (t.n_fill) {
      fill_seed = t.fill_seed;
      fill_seed_set = true;
    }
    for (int32_t j = 0; j < t.n_fill; j++)
      if (t.fill_pages[j] < 0 || t.fill_pages[j] >= d->p->physical_pages)
        return fail(s, RSTR_E_INVALID, "staged fill page out of range");
    for (int32_t j = 0; j < 2 * t.n_cow; j++)
      if (t.cow_pairs[j] < 0 || t.cow_pairs[j] >= d->p->physical_pages)
        return fail(s, RSTR_E_INVALID, "staged copy page out of range");
    words += d->desc_words;
    pages += t.n_fill + 2 * t.n_cow + 2 * t.n_prime;
  }
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  if (fill_seed_set) HIPCHK(s, ensure_templates(d->p, fill_seed));
  if (words > d->sched_desc_cap) {
    if (d->sched_desc) hipFree(d->sched_desc);
    d->sched_desc = nullptr;
    HIPCHK(s, dmalloc(&d->sched_desc, (size_t)words));
    d->sched_desc_cap = words;
  }
  if (pages > d->sched_pages_cap) {
    if (d->sched_pages) hipFree(d->sched_pages);
    d->sched_pages = nullptr;
    HIPCHK(s, dmalloc(&d->sched_pages, (size_t)std::max<int64_t>(pages, 1)));
    d->sched_pages_cap = pages;
  }
  if ((int64_t)n * d->B > d->sched_tok_cap) {
    if (d->sched_tok) hipFree(d->sched_tok);
    d->sched_tok = nullptr;
    HIPCHK(s, dmalloc(&d->sched_tok, (size_t)n * d->B));
    d->sched_tok_cap = (int64_t)n * d->B;
  }
  std::vector<int32_t> hdesc((size_t)words), hpages((size_t)std::max<int64_t>(pages, 1));
  d->sched.clear();
  int64_t wo = 0, po = 0;
  for (int32_t i = 0; i < n; i++) {
    const auto& t = steps[i];
    StagedDev sd{};
    sd.desc_off = wo;
    pack_desc(d, hdesc.data() + wo, t.slots, t.row_offsets, t.positions, t.page_table, t.lengths,
              t.start_positions);
    wo += d->desc_words;
    sd.fill_off = po;
    sd.n_fill = t.n_fill;
    sd.fill_seed = t.fill_seed;
    std::memcpy(hpages.data() + po, t.fill_pages, sizeof(int32_t) * t.n_fill);
    po += t.n_fill;
    sd.cow_off = po;
    sd.n_cow = t.n_cow;
    std::memcpy(hpages.data() + po, t.cow_pairs, sizeof(int32_t) * 2 * t.n_cow);
    po += 2 * t.n_cow;
    sd.prime_off = po;
    sd.n_prime = t.n_prime;
    sd.fused = fused_steps[i];
    std::memcpy(hpages.data() + po, t.prime_lanes, sizeof(int32_t) * t.n_prime);
    std::memcpy(hpages.data() + po + t.n_prime, t.prime_tokens, sizeof(int32_t) * t.n_prime);
    po += 2 * t.n_prime;
    d->sched.push_back(sd);
  }
  HIPCHK(s, hipMemcpy(d->sched_desc, hdesc.data(), sizeof(int32_t) * words, hipMemcpyHostToDevice));
  if (pages) HIPCHK(s, hipMemcpy(d->sched_pages, hpages.data(), sizeof(int32_t) * pages, hipMemcpyHostToDevice));
  return RSTR_OK;
}

static int sched_range(rstr_decoder* d, int32_t first, int32_t count) {
  if (first < 0 || count <= 0 || (size_t)first + count > d->sched.size())
    return fail(d->m->s, RSTR_E_INVALID, "schedule range out of bounds");
  return RSTR_OK;
}

static hipError_t enqueue_staged_prelude(rstr_decoder* d, const StagedDev& sd, hipStream_t st) {
  hipError_t e = hipSuccess;
  if (sd.n_fill)
    e = launch_fill_synthetic(st, d->p->d_slabs, d->m->d.n_layers, d->p->page_elems, d->p->tmpl,
                              d->sched_pages + sd.fill_off, sd.n_fill, sd.fill_seed);
  if (e == hipSuccess && sd.n_cow)
    e = launch_copy_pages(st, d->p->d_slabs, 2 * d->m->d.n_layers, d->p->page_elems,
                          d->sched_pages + sd.cow_off, sd.n_cow);
  if (e == hipSuccess && sd.n_prime)
    e = launch_gather_rows(st, d->m->emb, d->m->d.d_model, d->sched_pages + sd.prime_off,
                           d->sched_pages + sd.prime_off + sd.n_prime, sd.n_prime, d->r0);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d->desc, d->sched_desc + sd.desc_off, sizeof(int32_t) * d->desc_words,
                       hipMemcpyDeviceToDevice, st);
  return e;
}

extern "C" int rstr_schedule_run(rstr_decoder* d, int32_t first, int32_t count, int32_t* tokens_out,
                                 float* device_ms) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  int rc = sched_range(d, first, count);
  if (rc) return rc;
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  hipEvent_t a, b;
  HIPCHK(s, hipEventCreate(&a));
  HIPCHK(s, hipEventCreate(&b));
  HIPCHK(s, hipEventRecord(a, s->stream));
  for (int32_t i = first; i < first + count; i++) {
    HIPCHK(s, enqueue_staged_prelude(d, d->sched[i], s->stream));
    if ((rc = run_step_device(d, d->sched[i].fused))) return rc;
    HIPCHK(s, hipMemcpyAsync(d->sched_tok + (size_t)i * d->B, d->tokbuf, sizeof(int32_t) * d->B,
                             hipMemcpyDeviceToDevice, s->stream));
  }
  HIPCHK(s, hipEventRecord(b, s->stream));
  HIPCHK(s, hipEventSynchronize(b));
  float ms = 0.0f;
  HIPCHK(s, hipEventElapsedTime(&ms, a, b));
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (device_ms) *device_ms = ms;
  if (tokens_out)
    HIPCHK(s, hipMemcpy(tokens_out, d->sched_tok + (size_t)first * d->B, sizeof(int32_t) * count * d->B,
                        hipMemcpyDeviceToHost));
  return RSTR_OK;
}

extern "C" int rstr_decoder_profile_steps(rstr_decoder* d, int32_t first, int32_t count, float* class_ms,
                                          int32_t* class_launches) {
  if (!d) return fail(nullptr, RSTR_E_INVALID, "null decoder");
  rstr_session* s = d->m->s;
  int rc = sched_range(d, first, count);
  if (rc) return rc;
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, hipStreamSynchronize(s->stream));
  std::vector<double> acc(RSTR_K_CLASSES, 0.0);
  std::vector<int32_t> cnt(RSTR_K_CLASSES, 0);
  for (int32_t i = first; i < first + count; i++) {
    Prof prof;
    HIPCHK(s, enqueue_staged_prelude(d, d->sched[i], s->stream));
    HIPCHK(s, enqueue_step(d, s->stream, &prof, d->sched[i].fused));
    HIPCHK(s, hipStreamSynchronize(s->stream));
    for (auto& mk : prof.marks) {
      float ms = 0.0f;
      HIPCHK(s, hipEventElapsedTime(&ms, mk.second.first, mk.second.second));
      acc[mk.first] += ms;
      cnt[mk.first] += 1;
    }
  }
  d->has_logits = true;
  for (int c = 0; c < RSTR_K_CLASSES; c++) {
    if (class_ms) class_ms[c] = (float)acc[c];
    if (class_launches) class_launches[c] = cnt[c];
  }
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// isolated routed append
// ---------------------------------------------------------------------------
extern "C" int rstr_append_run(rstr_pool* p, int32_t layer, int32_t batch, const float* k_rows,
                               const float* v_rows, const int32_t* slots) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  const auto& md = p->m->d;
  if (layer < 0 || layer >= md.n_layers) return fail(s, RSTR_E_INVALID, "Paged append layer is outside its state slab");
  if (batch <= 0) return fail(s, RSTR_E_INVALID, "Paged append capacity must be a positive integer");
  if (!k_rows || !v_rows || !slots) return fail(s, RSTR_E_INVALID, "null append input");
  int64_t limit = (int64_t)p->physical_pages * p->page_size;
  std::vector<int32_t> seen;
  for (int b = 0; b < batch; b++) {
    if (slots[b] < -1 || slots[b] >= limit) return fail(s, RSTR_E_INVALID, "append slot out of range");
    if (slots[b] >= 0) seen.push_back(slots[b]);
  }
  std::sort(seen.begin(), seen.end());
  if (std::adjacent_find(seen.begin(), seen.end()) != seen.end())
    return fail(s, RSTR_E_INVALID, "append slots must be distinct");
  int kvr = md.n_kv * md.head_dim;
  float *dk = nullptr, *dv = nullptr;
  int32_t* ds = nullptr;
  HIPCHK(s, hipSetDevice(s->device));
  hipError_t e = dmalloc(&dk, (size_t)batch * kvr);
  if (e == hipSuccess) e = dmalloc(&dv, (size_t)batch * kvr);
  if (e == hipSuccess) e = dmalloc(&ds, (size_t)batch);
  if (e == hipSuccess) e = hipMemcpy(dk, k_rows, sizeof(float) * batch * kvr, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dv, v_rows, sizeof(float) * batch * kvr, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(ds, slots, sizeof(int32_t) * batch, hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = launch_append_rows(s->stream, dk, dv, batch, kvr, ds, p->slabs[layer], p->slabs[md.n_layers + layer]);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  if (dk) hipFree(dk);
  if (dv) hipFree(dv);
  if (ds) hipFree(ds);
  HIPCHK(s, e);
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// isolated decode tail
// ---------------------------------------------------------------------------
extern "C" int rstr_tail_run(rstr_session* s, int32_t rows, int32_t vocab, int32_t d, const float* logits,
                             const float* emb, int32_t* tokens_out, float* rows_out) {
  if (!s) return fail(nullptr, RSTR_E_INVALID, "null session");
  if (rows <= 0 || vocab <= 0 || d <= 0) return fail(s, RSTR_E_INVALID, "tail extents must be positive");
  if (!logits || !emb || !tokens_out || !rows_out) return fail(s, RSTR_E_INVALID, "null tail buffer");
  HIPCHK(s, hipSetDevice(s->device));
  float *dl = nullptr, *de = nullptr, *dr = nullptr;
  int32_t *dt = nullptr, *dc = nullptr;
  hipError_t e = dmalloc(&dl, (size_t)rows * vocab);
  if (e == hipSuccess) e = dmalloc(&de, (size_t)vocab * d);
  if (e == hipSuccess) e = dmalloc(&dr, (size_t)rows * d);
  if (e == hipSuccess) e = dmalloc(&dt, (size_t)rows);
  if (e == hipSuccess) e = dmalloc(&dc, (size_t)2 * rows * argmax_segments(rows, vocab));
  if (e == hipSuccess) e = hipMemcpy(dl, logits, sizeof(float) * rows * vocab, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(de, emb, sizeof(float) * vocab * d, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_argmax_gather(s->stream, dl, rows, vocab, de, d, dt, dr, dc);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  if (e == hipSuccess) e = hipMemcpy(tokens_out, dt, sizeof(int32_t) * rows, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemcpy(rows_out, dr, sizeof(float) * rows * d, hipMemcpyDeviceToHost);
  for (void* q : {(void*)dl, (void*)de, (void*)dr, (void*)dt, (void*)dc})
    if (q) hipFree(q);
  HIPCHK(s, e);
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// isolated dequantising linear (kernel-level parity of every projection form)
// ---------------------------------------------------------------------------
extern "C" int rstr_linear_run(rstr_model* m, int32_t layer, int32_t role, int32_t rows, const int8_t* xq,
                               const float* xs, int32_t splits, int32_t form, float* y) {
  if (!m) return fail(nullptr, RSTR_E_INVALID, "null model");
  rstr_session* s = m->s;
  if (!xq || !xs || !y) return fail(s, RSTR_E_INVALID, "null linear buffer");
  const QTensor* t = nullptr;
  if (role == RSTR_ROLE_EMBED) t = &m->head;
  else if (layer >= 0 && layer < (int32_t)m->layers.size()) {
    LayerW& L = m->layers[layer];
    if (role == RSTR_ROLE_Q) t = &L.qkv;
    else if (role == RSTR_ROLE_O) t = &L.o;
    else if (role == RSTR_ROLE_GATE) t = &L.gu;
    else if (role == RSTR_ROLE_DOWN) t = &L.down;
  }
  if (!t) return fail(s, RSTR_E_INVALID, "no such linear (roles: embed, q = fused qkv, o, gate = fused gate/up, down)");
  if (rows < 1 || rows > 4096) return fail(s, RSTR_E_INVALID, "rows must be in [1, 4096]");
  if (splits != 1 && splits != 2 && splits != 4) return fail(s, RSTR_E_INVALID, "splits must be 1, 2 or 4");
  if (form < QG_FORM_AUTO || form > QG_FORM_WG_GEMV) return fail(s, RSTR_E_INVALID, "unknown projection form");
  const int K = t->k, N = t->n, nb = K / 32, mpad = (rows + 15) / 16 * 16;
  // activation operand in the MFMA tile order: fp16 q*d [mpad/16][nb][g][m%16][8]
  // (exact: d has a 4-bit significand), scales [nb][mpad]; padding rows are 0
  std::vector<_Float16> hq((size_t)mpad * K, (_Float16)0.0f);
  std::vector<float> hs((size_t)nb * mpad, 0.0f);
  for (int r = 0; r < rows; r++)
    for (int b = 0; b < nb; b++) {
      const float d = xs[(size_t)r * nb + b];
      hs[(size_t)b * mpad + r] = d;
      for (int g = 0; g < 4; g++)
        for (int e = 0; e < 8; e++)
          hq[((((size_t)(r >> 4) * nb + b) * 4 + g) * 16 + (r & 15)) * 8 + e] =
              (_Float16)((float)xq[(size_t)r * K + 32 * b + 8 * g + e] * d);
    }
  HIPCHK(s, hipSetDevice(s->device));
  ActBuf x;
  x.mpad = mpad;
  float* dy = nullptr;
  hipError_t e = dmalloc(&x.q, hq.size());
  if (e == hipSuccess) e = dmalloc(&x.s, hs.size());
  if (e == hipSuccess) e = dmalloc(&dy, (size_t)splits * rows * N);
  if (e == hipSuccess) e = hipMemcpy(x.q, hq.data(), hq.size() * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(x.s, hs.data(), hs.size() * 4, hipMemcpyHostToDevice);
  hipError_t le = hipSuccess;
  if (e == hipSuccess) {
    le = launch_qgemm_form(s->stream, *t, x, rows, dy, N, splits, (size_t)rows * N, form);
    if (le == hipSuccess) e = hipStreamSynchronize(s->stream);
  }
  std::vector<float> sl((size_t)splits * rows * N);
  if (e == hipSuccess && le == hipSuccess) e = hipMemcpy(sl.data(), dy, sl.size() * 4, hipMemcpyDeviceToHost);
  for (void* q : {(void*)x.q, (void*)x.s, (void*)dy})
    if (q) hipFree(q);
  if (le == hipErrorInvalidValue) return fail(s, RSTR_E_INVALID, "the projection form does not serve this shape");
  HIPCHK(s, le);
  HIPCHK(s, e);
  // slices in the consumers' canonical tree: (s0 + s1) or ((s0 + s1) + (s2 + s3))
  const size_t n = (size_t)rows * N;
  for (size_t i = 0; i < n; i++) {
    if (splits == 1) y[i] = sl[i];
    else if (splits == 2) y[i] = sl[i] + sl[n + i];
    else y[i] = (sl[i] + sl[n + i]) + (sl[2 * n + i] + sl[3 * n + i]);
  }
  return RSTR_OK;
}

// ---------------------------------------------------------------------------
// isolated routed attention
// ---------------------------------------------------------------------------
struct AttnBufs {
  float *q = nullptr, *out = nullptr, *part = nullptr;
  int32_t *pt = nullptr, *len = nullptr, *tab = nullptr;
  ~AttnBufs() {
    for (void* p : {(void*)q, (void*)out, (void*)part, (void*)pt, (void*)len, (void*)tab})
      if (p) hipFree(p);
  }
};

// Checks shared by the isolated attention entries; returns the longest route.
static int attn_validate(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split, int32_t window,
                         const float* q, const int32_t* pt, int32_t pps, const int32_t* len, int64_t* maxlen) {
  rstr_session* s = p->m->s;
  const auto& md = p->m->d;
  if (layer < 0 || layer >= md.n_layers) return fail(s, RSTR_E_INVALID, "layer out of range");
  if (batch <= 0 || pps <= 0 || n_q <= 0 || n_q % md.n_kv)
    return fail(s, RSTR_E_INVALID, "Paged-attention capacity must be a positive integer");
  int G = n_q / md.n_kv;
  if (G != 1 && G != 2 && G != 4 && G != 8) return fail(s, RSTR_E_INVALID, "unsupported GQA group");
  if (split <= 0 || split % 4 || split > 4096) return fail(s, RSTR_E_INVALID, "invalid split");
  if (window < 0) return fail(s, RSTR_E_INVALID, "invalid window");
  if (!q || !pt || !len) return fail(s, RSTR_E_INVALID, "null attention input");
  int ps = p->page_size;
  *maxlen = 0;
  for (int b = 0; b < batch; b++) {
    if (len[b] < 0 || (int64_t)len[b] > (int64_t)pps * ps) return fail(s, RSTR_E_INVALID, "length out of range");
    for (int i = 0; i < (len[b] + ps - 1) / ps; i++) {
      int32_t pg = pt[(int64_t)b * pps + i];
      if (pg < 0 || pg >= p->physical_pages) return fail(s, RSTR_E_INVALID, "page table entry out of range");
    }
    *maxlen = std::max<int64_t>(*maxlen, len[b]);
  }
  return RSTR_OK;
}

static int attn_prepare(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split,
                        int32_t window, const float* q, const int32_t* pt, int32_t pps,
                        const int32_t* len, AttnBufs& bf, AttnGeom& geo, int* max_items) {
  rstr_session* s = p->m->s;
  const auto& md = p->m->d;
  int64_t maxlen = 0;
  int rc = attn_validate(p, layer, batch, n_q, split, window, q, pt, pps, len, &maxlen);
  if (rc) return rc;
  int G = n_q / md.n_kv;
  int hd = md.head_dim;
  *max_items = (int)std::max<int64_t>(1, (int64_t)batch * md.n_kv * ((maxlen + split - 1) / split + 1));
  HIPCHK(s, hipSetDevice(s->device));
  HIPCHK(s, dmalloc(&bf.q, (size_t)batch * n_q * hd));
  HIPCHK(s, dmalloc(&bf.out, (size_t)batch * n_q * hd));
  HIPCHK(s, dmalloc(&bf.part, (size_t)*max_items * G * attn_part_floats(hd)));
  HIPCHK(s, dmalloc(&bf.pt, (size_t)batch * pps));
  HIPCHK(s, dmalloc(&bf.len, (size_t)batch));
  geo = AttnGeom{batch, n_q, md.n_kv, hd, p->page_size, pps, split, window, 0.0f};
  const size_t tabw = attn_tab_words(geo, *max_items);
  if (tabw == 0) return fail(s, RSTR_E_INVALID, "unsupported attention geometry");
  HIPCHK(s, dmalloc(&bf.tab, tabw));
  HIPCHK(s, hipMemcpy(bf.q, q, sizeof(float) * batch * n_q * hd, hipMemcpyHostToDevice));
  HIPCHK(s, hipMemcpy(bf.pt, pt, sizeof(int32_t) * batch * pps, hipMemcpyHostToDevice));
  HIPCHK(s, hipMemcpy(bf.len, len, sizeof(int32_t) * batch, hipMemcpyHostToDevice));
  return RSTR_OK;
}

static int attn_check_rows(rstr_session* s, int32_t batch, const int32_t* row_offsets, const int32_t* positions,
                           const int32_t* lengths, const int32_t* start_positions, float* out) {
  if (!row_offsets || !positions || !start_positions || !out)
    return fail(s, RSTR_E_INVALID, "null attention descriptor");
  for (int b = 0; b <= batch; b++)
    if (row_offsets[b] != b) return fail(s, RSTR_E_INVALID, "row offsets must be 0..batch");
  for (int b = 0; b < batch; b++) {
    if (start_positions[b] < 0) return fail(s, RSTR_E_INVALID, "Resident route identity and extents are invalid");
    if (lengths && lengths[b] > 0 && (int64_t)positions[b] != (int64_t)start_positions[b] + lengths[b] - 1)
      return fail(s, RSTR_E_INVALID, "query position must be the route's last visible token");
  }
  return RSTR_OK;
}

extern "C" int rstr_attention_run(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split,
                                  int32_t window, float scale, const float* q, const int32_t* row_offsets,
                                  const int32_t* positions, const int32_t* page_table, int32_t pps,
                                  const int32_t* lengths, const int32_t* start_positions, float* out) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  int rc = attn_check_rows(s, batch, row_offsets, positions, lengths, start_positions, out);
  if (rc) return rc;
  AttnBufs bf;
  AttnGeom geo;
  int max_items = 0;
  rc = attn_prepare(p, layer, batch, n_q, split, window, q, page_table, pps, lengths, bf, geo, &max_items);
  if (rc) return rc;
  geo.scale = scale;
  hipStream_t st = s->stream;
  int L = p->m->d.n_layers;
  HIPCHK(s, launch_attn_lists(st, &geo, 1, bf.len, bf.tab, 0, max_items));
  HIPCHK(s, launch_attn_split(st, geo, bf.q, p->slabs[layer], p->slabs[L + layer], bf.pt, bf.tab, bf.part,
                              max_items));
  HIPCHK(s, launch_attn_merge(st, geo, bf.len, bf.tab, bf.part, bf.out, nullptr));
  HIPCHK(s, hipStreamSynchronize(st));
  HIPCHK(s, hipMemcpy(out, bf.out, sizeof(float) * batch * n_q * geo.hd, hipMemcpyDeviceToHost));
  return RSTR_OK;
}

// The same attention with every device buffer carved out of the session GPU's
// static staging array (256-byte aligned regions); the work list is sized to
// the routes' exact item count, which changes only how items are spread over
// waves, never an item's arithmetic.
extern "C" int rstr_attention_run_static(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split,
                                         int32_t window, float scale, const float* q, const int32_t* row_offsets,
                                         const int32_t* positions, const int32_t* page_table, int32_t pps,
                                         const int32_t* lengths, const int32_t* start_positions, float* out) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  int rc = attn_check_rows(s, batch, row_offsets, positions, lengths, start_positions, out);
  if (rc) return rc;
  int64_t maxlen = 0;
  if ((rc = attn_validate(p, layer, batch, n_q, split, window, q, page_table, pps, lengths, &maxlen))) return rc;
  const auto& md = p->m->d;
  const int hd = md.head_dim, G = n_q / md.n_kv;
  // exact item count: n_kv items per split of each lane's visible range
  int64_t items = 0;
  for (int b = 0; b < batch; b++) {
    const int64_t L = lengths[b];
    if (L <= 0) continue;
    const int64_t lo = window > 0 ? std::max<int64_t>(0, L - window) : 0;
    items += (int64_t)md.n_kv * ((L - 1) / split - lo / split + 1);
  }
  items = std::max<int64_t>(items, 1);
  if (items > INT32_MAX / 4) return fail(s, RSTR_E_INVALID, "attention work exceeds the static staging maximum");
  const int max_items = (int)items;
  AttnGeom geo{batch, n_q, md.n_kv, hd, p->page_size, pps, split, window, scale};
  const size_t tabw = attn_tab_words(geo, max_items);
  if (tabw == 0) return fail(s, RSTR_E_INVALID, "unsupported attention geometry");
  auto al = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
  const size_t qb = sizeof(float) * (size_t)batch * n_q * hd, ptb = sizeof(int32_t) * (size_t)batch * pps,
               lb = sizeof(int32_t) * (size_t)batch, tb = sizeof(int32_t) * tabw,
               pb = sizeof(float) * (size_t)max_items * G * attn_part_floats(hd);
  const size_t o_q = 0, o_out = o_q + al(qb), o_pt = o_out + al(qb), o_len = o_pt + al(ptb), o_tab = o_len + al(lb),
               o_part = o_tab + al(tb), total = o_part + al(pb);
  if (total > (size_t)RSTR_ATTN_STATIC_BYTES)
    return fail(s, RSTR_E_INVALID, "attention staging of " + std::to_string(total) +
                                       " bytes exceeds the static staging maximum of " +
                                       std::to_string((long long)RSTR_ATTN_STATIC_BYTES) + " bytes");
  HIPCHK(s, hipSetDevice(s->device));
  char* base = static_cast<char*>(s->scratch);
  float* dq = reinterpret_cast<float*>(base + o_q);
  float* dout = reinterpret_cast<float*>(base + o_out);
  int32_t* dpt = reinterpret_cast<int32_t*>(base + o_pt);
  int32_t* dlen = reinterpret_cast<int32_t*>(base + o_len);
  int32_t* dtab = reinterpret_cast<int32_t*>(base + o_tab);
  float* dpart = reinterpret_cast<float*>(base + o_part);
  hipStream_t st = s->stream;
  const int L = md.n_layers;
  // the previous call on this session finished before it returned; the copies
  // complete before the kernels that read them are launched
  HIPCHK(s, hipMemcpy(dq, q, qb, hipMemcpyHostToDevice));
  HIPCHK(s, hipMemcpy(dpt, page_table, ptb, hipMemcpyHostToDevice));
  HIPCHK(s, hipMemcpy(dlen, lengths, lb, hipMemcpyHostToDevice));
  HIPCHK(s, launch_attn_lists(st, &geo, 1, dlen, dtab, 0, max_items));
  HIPCHK(s, launch_attn_split(st, geo, dq, p->slabs[layer], p->slabs[L + layer], dpt, dtab, dpart, max_items));
  HIPCHK(s, launch_attn_merge(st, geo, dlen, dtab, dpart, dout, nullptr));
  HIPCHK(s, hipStreamSynchronize(st));
  HIPCHK(s, hipMemcpy(out, dout, qb, hipMemcpyDeviceToHost));
  return RSTR_OK;
}

extern "C" int rstr_attention_bench(rstr_pool* p, int32_t layer, int32_t batch, int32_t n_q, int32_t split,
                                    int32_t window, float scale, const float* q, const int32_t* page_table,
                                    int32_t pps, const int32_t* lengths, int32_t iters, float* split_ms,
                                    float* merge_ms) {
  if (!p) return fail(nullptr, RSTR_E_INVALID, "null pool");
  rstr_session* s = p->m->s;
  if (iters <= 0) return fail(s, RSTR_E_INVALID, "iters must be positive");
  AttnBufs bf;
  AttnGeom geo;
  int max_items = 0;
  int rc = attn_prepare(p, layer, batch, n_q, split, window, q, page_table, pps, lengths, bf, geo, &max_items);
  if (rc) return rc;
  geo.scale = scale;
  hipStream_t st = s->stream;
  int L = p->m->d.n_layers;
  HIPCHK(s, launch_attn_lists(st, &geo, 1, bf.len, bf.tab, 0, max_items));
  std::vector<hipEvent_t> ev(4 * iters);
  for (auto& e : ev) HIPCHK(s, hipEventCreate(&e));
  for (int i = 0; i < iters; i++) {
    HIPCHK(s, hipEventRecord(ev[4 * i], st));
    HIPCHK(s, launch_attn_split(st, geo, bf.q, p->slabs[layer], p->slabs[L + layer], bf.pt, bf.tab, bf.part,
                                max_items));
    HIPCHK(s, hipEventRecord(ev[4 * i + 1], st));
    HIPCHK(s, hipEventRecord(ev[4 * i + 2], st));
    HIPCHK(s, launch_attn_merge(st, geo, bf.len, bf.tab, bf.part, bf.out, nullptr));
    HIPCHK(s, hipEventRecord(ev[4 * i + 3], st));
  }
  HIPCHK(s, hipStreamSynchronize(st));
  double ssum = 0, msum = 0;
  for (int i = 0; i < iters; i++) {
    float a = 0, b = 0;
    HIPCHK(s, hipEventElapsedTime(&a, ev[4 * i], ev[4 * i + 1]));
    HIPCHK(s, hipEventElapsedTime(&b, ev[4 * i + 2], ev[4 * i + 3]));
    ssum += a;
    msum += b;
  }
  for (auto& e : ev) hipEventDestroy(e);
  if (split_ms) *split_ms = (float)(ssum / iters);
  if (merge_ms) *merge_ms = (float)(msum / iters);
  return RSTR_OK;
}

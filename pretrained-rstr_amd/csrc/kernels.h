// kernels.h -- host-side launch interface of the gfx950 decode-step kernels.
//
// Device data layouts (all chosen for 128-bit coalesced loads on CDNA4):
//
//  Quantised linear W[N][K] (N % 16 == 0, K % 128 == 0, nb = K/32 blocks):
//   column tile ct = n/16, block group bq = b/4, k-group g = (k%32)/8,
//   lane column nn = n%16, block-in-group bb = b%4.
//   Q4 dword  [ct][bq][g][nn][bb]  holds the 8 nibbles of weights
//             k = 32b + 8g + {0..7}; nibble i carries k_local = {0,2,4,6,1,3,5,7}[i].
//   Q8 dwords [ct][bq][g][nn][bb][2]; byte i carries k_local = {0,2,1,3,4,6,5,7}[i].
//   fp16 scales [ct][bq][nn/4][bb][nn%4] (a lane whose accumulator holds
//   columns 4j..4j+3 of a tile reads its 4 blocks' scales as one 32-byte run).
//   (These permutations make the nibble/byte -> fp16 expansion a mask-or plus
//   one packed fp16 add; the canonical row-major order is restored on export.)
//
//  Quantised activation X[M][K] for the MFMA B operand (Mpad = 16*ceil(M/16)):
//   fp16 values q*d [Mpad/16][nb][g][m%16][8] (exact: the block scale d has a
//   4-bit significand), fp32 block scales d [nb][Mpad].
//
//  KV pages per layer and slab: fp16 [page][page_size][n_kv][head_dim]
//   (the routed-append ABI of doc/serving-architecture.md:178-190).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rstr {

struct QTensor {       // one device-resident quantised matrix
  void* w = nullptr;   // packed dwords
  uint16_t* s = nullptr;
  int n = 0, k = 0, bits = 4;
};

struct ActBuf {        // quantised activations in MFMA tile order
  _Float16* q = nullptr; // q*d per element
  float* s = nullptr;    // d per (block, row)
  int mpad = 0;
};

// weights
hipError_t launch_gen_linear(hipStream_t st, const QTensor& t, int col_off, int n_rows, int k,
                             uint64_t key, const float* src_f32);
hipError_t launch_gen_f32(hipStream_t st, float* out, int64_t n, uint64_t key, double mean,
                          double std, double scale);
hipError_t launch_prescale(hipStream_t st, float* out, const float* in, int64_t n, double scale);

// projections.  A projection whose K range is split over S workgroups writes S
// output slices `stride` floats apart; consumers combine them in the canonical
// tree order, (s0+s1) or ((s0+s1)+(s2+s3)).
struct Slices {
  const float* p;
  int n;
  size_t stride;
};
int qgemm_splits(int n, int mpad, int bits);
hipError_t launch_qgemm(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y,
                        int ldy, int splits, size_t slice_stride);
// Gate/up (w = [gate | up], n = 2*ff) with act(gate)*up quantised into `out`
// in the epilogue (the fp32 gate/up output is not written); the same bits as
// launch_qgemm + launch_act_quant.  qgemm_act_fused says where it is used.
bool qgemm_act_fused(int ff, int mpad);
hipError_t launch_qgemm_act(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, int ff, int geglu,
                            ActBuf& out);
// The same projection with the kernel form chosen by the caller (kernel-level
// parity tests): AUTO is launch_qgemm's own choice; TILE the MFMA tile plan;
// WAVE_GEMV / WG_GEMV the weight-streaming GEMVs (m_rows <= 4).  A form that
// does not serve the shape returns hipErrorInvalidValue before any device work.
enum { QG_FORM_AUTO = 0, QG_FORM_TILE = 1, QG_FORM_WAVE_GEMV = 2, QG_FORM_WG_GEMV = 3 };
hipError_t launch_qgemm_form(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy,
                             int splits, size_t slice_stride, int form);
// The down projection with its input computed in the projection itself: at
// one to four rows, where launch_qgemm runs a weight-streaming GEMV, the
// activation gate (launch_act_quant) folds into the GEMV's staging of its
// activations -- hh = act(gate) * up from the gate/up slices of the
// workgroup's K range, its 32-block scale and integers by the rule of
// launch_act_quant, so the bits equal launch_act_quant followed by
// launch_qgemm.  Returns hipErrorNotSupported, before any device work, for any
// other shape (the caller then launches the two kernels).
struct ActIn {
  const float* gu;   // gate/up output slices [S][rows][2*ff] (gate | up)
  size_t stride;     // floats between slices
  int S, ff, geglu;
};
hipError_t launch_qgemm_actin(hipStream_t st, const QTensor& w, const ActIn& ain, int mpad, int m_rows, float* y,
                              int ldy, int splits, size_t slice_stride);
// Few-row weight-streaming GEMVs (m_rows <= 4; launch_qgemm picks them per
// shape): one wave per (column tile, split), or one workgroup per (column
// tile, split) whose waves share the split's 4-block groups.
hipError_t launch_qgemv(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy,
                        int splits, size_t slice_stride);
hipError_t launch_qgemv_wg(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy,
                           int splits, size_t slice_stride);

// row kernels
hipError_t launch_rms_quant(hipStream_t st, const float* x, const float* g, float goff, float eps,
                            int rows, int n, ActBuf& out);
hipError_t launch_post_attn(hipStream_t st, Slices o, const float* x, float* xmid,
                            const float* paln, const float* pfln, float goff, float eps, int rows,
                            int n, ActBuf& out);
hipError_t launch_post_ffn(hipStream_t st, Slices dn, const float* xmid, float* xout,
                           const float* pffln, const float* gnext, float goff, float eps, int rows,
                           int n, ActBuf& out);
hipError_t launch_act_quant(hipStream_t st, Slices gu, int rows, int ff, int geglu,
                            ActBuf& out);
hipError_t launch_qkv_post(hipStream_t st, Slices yqkv, int rows, int n_q, int n_kv, int hd,
                           const float* qn, const float* kn, float goff, float eps,
                           const float* cos_t, const float* sin_t, const int32_t* positions,
                           const int32_t* slots, float* qr, uint16_t* kpages, uint16_t* vpages);

// attention
struct AttnGeom {
  int batch, n_q, n_kv, hd, page_size, pps, split, window;
  float scale;
};
// Attention work table of one step and window geometry (int32 words):
//   lo[B] k0[B] nsplit[B] base[B+1] fbase[B+1] pbase[B+1]   per lane (window
//       start, first split, split count, and prefixes of its items, full
//       items and partial items);
//   ctr arm          the split kernel's claim counter and the value that arms
//       it (written by the prep, re-armed by the merge after every split);
//   boff[RSTR_NCH] cur[RSTR_NCH]   partial items by chunk count: list offset
//       of each count (larger counts first) and the fill cursor of each;
//   items[max_items][4] at a 16-byte boundary: the work list, full items then
//       partial ones by decreasing chunk count, entries
//       (lane | kv head << 20, t0, t1, item index).
// max_items bounds the step's items (sum over lanes of n_kv * splits).
#define RSTR_NCH 260  // chunk counts of one split (split <= 4096 tokens)
// Split partial of one (item, query head): o[hd], m, l and two pad floats, so
// every record starts on a 16-byte boundary.  An item holds G such records.
__host__ __device__ constexpr int attn_part_floats(int hd) { return hd + 4; }
__host__ __device__ inline int attn_ctl_offset(int batch) { return 6 * batch + 3; }
__host__ __device__ inline int attn_bucket_offset(int batch) { return 6 * batch + 5; }
// Static rounds of an n-item work list over R split waves: every round when
// the list fits in two, else at least two and all but the last one to two
// (those are claimed from a counter armed to the returned value times R).
__host__ __device__ inline int attn_static_rounds(int n, int R) {
  const int c = (n + R - 1) / R;
  if (c <= 2) return c;
  return n / R - 1 > 2 ? n / R - 1 : 2;
}
inline int lane_tab_words(int batch) { return 6 * batch + 5 + 2 * RSTR_NCH; }
inline size_t attn_items_offset(int batch) { return ((size_t)lane_tab_words(batch) + 3) & ~(size_t)3; }
int attn_grid(const AttnGeom& g, int max_items);              // 0: unsupported geometry
size_t attn_tab_words(const AttnGeom& g, int max_items);      // 0: unsupported geometry
hipError_t launch_attn_prep(hipStream_t st, const AttnGeom& g, const int32_t* lengths,
                            int32_t* lane_tab, int max_items);
// The work lists of n_geo (1 or 2) geometries that share batch, split and
// lengths (lane tables `tab_stride` words apart): one launch for batches of
// up to 1024 lanes.
hipError_t launch_attn_lists(hipStream_t st, const AttnGeom* g, int n_geo, const int32_t* lengths,
                             int32_t* lane_tab, size_t tab_stride, int max_items);
// The attention output written by the few-item split kernel itself, quantised
// for the output projection as k_attn_merge writes it (q*d in MFMA tile order,
// block scales [nb][mpad]).  Only for launches whose every lane's visible
// range is one split (a merge of one partial) and that run the few-item
// kernel (attn_direct_out); rows of lanes without items are left as they are.
struct AttnOut {
  _Float16* q;
  float* s;
  int mpad;
};
bool attn_direct_out(const AttnGeom& g, int max_items);
hipError_t launch_attn_split(hipStream_t st, const AttnGeom& g, const float* q,
                             const uint16_t* kpages, const uint16_t* vpages,
                             const int32_t* page_table, int32_t* lane_tab, float* part,
                             int max_items, const AttnOut* out = nullptr);
// The decode step's per-row qkv post-processing (launch_qkv_post) done by the
// few-item attention kernel instead of a launch of its own: each item computes
// its heads' q from the projection slices (qk-norm, RoPE at the row's position),
// and the item that holds a lane's newest token appends that token's K/V (fp16
// RNE) before its first page load.  Only valid when no lane's visible range
// holds another lane's appended slot (attn_fuses_qkv says when the few-item
// kernel runs; the caller checks the descriptors).
struct AttnQkv {
  Slices y;                          // qkv projection output in slices
  const float *qn, *kn;              // qk-norm gains (null: none)
  float goff, eps;
  const float *cos_t, *sin_t;        // [maxpos][hd/2] of the layer's theta
  const int32_t *positions, *slots, *lengths;
  uint16_t *kpages, *vpages;         // the layer's slabs (written at the slots)
};
bool attn_fuses_qkv(const AttnGeom& g, int max_items);
hipError_t launch_attn_split_qkv(hipStream_t st, const AttnGeom& g, const AttnQkv& qk,
                                 const int32_t* page_table, int32_t* lane_tab, float* part, int max_items,
                                 const AttnOut* out = nullptr);
hipError_t launch_attn_merge(hipStream_t st, const AttnGeom& g, const int32_t* lengths,
                             int32_t* lane_tab, const float* part, float* out_f32,
                             ActBuf* out_q);

// tail, priming, pages
// Segments per row of the tail's first stage; the candidate buffer holds
// rows * argmax_segments(rows, vocab) (value, index) pairs of int32 words.
int argmax_segments(int rows, int vocab);
hipError_t launch_argmax_gather(hipStream_t st, const float* logits, int rows, int vocab,
                                const float* emb, int d, int32_t* tok, float* r0, int32_t* cand);
hipError_t launch_gather_rows(hipStream_t st, const float* emb, int d, const int32_t* lanes,
                              const int32_t* tokens, int n, float* r0);
hipError_t launch_append_rows(hipStream_t st, const float* k_rows, const float* v_rows, int rows,
                              int kvr, const int32_t* slots, uint16_t* kpages, uint16_t* vpages);
hipError_t launch_copy_pages(hipStream_t st, uint16_t** slabs, int nslabs, int64_t page_elems,
                             const int32_t* pairs, int npairs);
// dtype 0: f32, 1: f16, 2: bf16 -> f32 (exact)
hipError_t launch_widen(hipStream_t st, int dtype, const void* src, float* dst, int64_t n);
// mode 0: pool -> fp16 payload; 1: fp16 payload -> pool; 2: f32 payload -> pool (RNE)
hipError_t launch_chunk_move(hipStream_t st, int mode, uint16_t** slabs, int nslabs, const int32_t* pages,
                             int start, int count, int page_size, int ept, void* payload);
// The allocation-free attention entry's staging array (one per GPU) and its
// device address on the current device (call once per device, device current).
#define RSTR_STATIC_SCRATCH_BYTES (64ll << 20)
hipError_t static_scratch_address(void** ptr);

#define RSTR_SYNTH_TEMPLATES 64
hipError_t launch_gen_templates(hipStream_t st, uint16_t* tmpl, int n_layers, int64_t page_elems,
                                uint64_t seed);
hipError_t launch_fill_synthetic(hipStream_t st, uint16_t** slabs, int n_layers,
                                 int64_t page_elems, const uint16_t* tmpl, const int32_t* pages,
                                 int npages, uint64_t seed);


}  // namespace rstr

// kernels.hip -- gfx950 kernels of the resident continuous decode step.
//
// Each kernel reproduces one op of the reference decode step
// (src/pretrained/decoder_gpu.clj:122-220 layer/head order, :64-91 tail)
// with the canonical fp32 operation order documented next to it, so the CPU
// restatement can check every intermediate bit-for-bit.
#include "device_math.h"
#include "kernels.h"

#include <climits>

namespace rstr {

// ===========================================================================
// Weight generation / quantisation
// ===========================================================================
// Q4 block (GGML Q4_0 rule): d = (signed max-magnitude)/-8,
// q = min(15, trunc(w/d + 8.5)); scale stored fp16.  Q8: d = max|w|/127,
// q = rint(w/d).  Source: device f32 matrix or the counter-based generator.
template <int BITS>
__global__ void k_gen_linear(uint32_t* __restrict__ W, uint16_t* __restrict__ S, int nb, int col_off,
                             int n_rows, int k, uint64_t key, const float* __restrict__ src) {
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)n_rows * nb) return;
  int n = (int)(gid / nb), b = (int)(gid % nb);
  float w[32];
  uint64_t base = (uint64_t)n * (uint64_t)k + (uint64_t)(32 * b);
#pragma unroll
  for (int i = 0; i < 32; i++)
    w[i] = src ? src[base + i] : synth_normal(key, base + (uint64_t)i, 0.0, 0.02);
  int ncat = col_off + n;
  int ct = ncat >> 4, nn = ncat & 15, bq = b >> 2, bb = b & 3, nb4 = nb >> 2;
  uint16_t scale;
  if (BITS == 4) {
    float amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
      float a = fabsf(w[i]);
      if (a > amax) { amax = a; mx = w[i]; }
    }
    // An all-zero block gets scale +0 (written as a select so no fused
    // multiply-convert can turn the sign of a zero product around).
    float d = (amax > 0.0f) ? mx / -8.0f : 0.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    uint32_t q[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
      int v = (int)(w[i] * id + 8.5f);
      q[i] = (uint32_t)(v > 15 ? 15 : v);
    }
    const int perm[8] = {0, 2, 4, 6, 1, 3, 5, 7};
#pragma unroll
    for (int g = 0; g < 4; g++) {
      uint32_t dw = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) dw |= q[8 * g + perm[i]] << (4 * i);
      W[((((size_t)ct * nb4 + bq) * 4 + g) * 16 + nn) * 4 + bb] = dw;
    }
    scale = f2h_bits(d);
  } else {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(w[i]));
    float d = amax / 127.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    int q[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
      int v = (int)__builtin_rintf(w[i] * id);
      q[i] = v > 127 ? 127 : (v < -127 ? -127 : v);
    }
    const int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
#pragma unroll
    for (int g = 0; g < 4; g++) {
      uint32_t d0 = 0, d1 = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        d0 |= ((uint32_t)q[8 * g + perm[i]] & 0xFFu) << (8 * i);
        d1 |= ((uint32_t)q[8 * g + perm[4 + i]] & 0xFFu) << (8 * i);
      }
      size_t idx = (((((size_t)ct * nb4 + bq) * 4 + g) * 16 + nn) * 4 + bb) * 2;
      W[idx] = d0;
      W[idx + 1] = d1;
    }
    scale = f2h_bits(d);
  }
  S[(((size_t)ct * nb4 + bq) * 16 + nn) * 4 + bb] = scale;
}

hipError_t launch_gen_linear(hipStream_t st, const QTensor& t, int col_off, int n_rows, int k,
                             uint64_t key, const float* src_f32) {
  int nb = k / 32;
  int64_t total = (int64_t)n_rows * nb;
  int threads = 256;
  int64_t blocks = (total + threads - 1) / threads;
  if (t.bits == 4)
    hipLaunchKernelGGL(k_gen_linear<4>, dim3((unsigned)blocks), dim3(threads), 0, st, (uint32_t*)t.w,
                       t.s, nb, col_off, n_rows, k, key, src_f32);
  else
    hipLaunchKernelGGL(k_gen_linear<8>, dim3((unsigned)blocks), dim3(threads), 0, st, (uint32_t*)t.w,
                       t.s, nb, col_off, n_rows, k, key, src_f32);
  return hipGetLastError();
}

// f32 synthetic vector; (float)(scale * (double)e) reproduces the double-math
// embedding prescale of decoder_gpu.clj:80-91 (scale = 1 leaves e unchanged).
__global__ void k_gen_f32(float* out, int64_t n, uint64_t key, double mean, double std, double scale) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float e = synth_normal(key, (uint64_t)i, mean, std);
  out[i] = (float)(scale * (double)e);
}

hipError_t launch_gen_f32(hipStream_t st, float* out, int64_t n, uint64_t key, double mean,
                          double std, double scale) {
  int threads = 256;
  int64_t blocks = (n + threads - 1) / threads;
  hipLaunchKernelGGL(k_gen_f32, dim3((unsigned)blocks), dim3(threads), 0, st, out, n, key, mean, std,
                     scale);
  return hipGetLastError();
}

__global__ void k_prescale(float* out, const float* in, int64_t n, double scale) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (float)(scale * (double)in[i]);
}

hipError_t launch_prescale(hipStream_t st, float* out, const float* in, int64_t n, double scale) {
  int threads = 256;
  int64_t blocks = (n + threads - 1) / threads;
  hipLaunchKernelGGL(k_prescale, dim3((unsigned)blocks), dim3(threads), 0, st, out, in, n, scale);
  return hipGetLastError();
}

// ===========================================================================
// Dequantising linear on MFMA: y[m][n] = sum_b isum(m,n,b) * (dw[n,b]*dx[m,b])
// ===========================================================================
// The block dot isum is computed exactly by v_mfma_f32_16x16x32_f16: both
// operands are small integers (|q_w| <= 8 or 127, |q_x| <= 127) held exactly
// in fp16, every partial sum is an integer below 2^24, so the fp32 result is
// the exact integer.  The block combination follows the canonical order:
// 64 contiguous parts of c = ceil(nb/64) blocks, acc = fmaf(isum, dw*dx, acc)
// in block order per part, parts combined by the balanced pairwise tree.
// Wave w of the workgroup owns parts [16w, 16w+16) (a complete level-4
// subtree, built with a binary-counter stack); the four subtrees meet in LDS
// as ((w0+w1)+(w2+w3)).

__device__ __forceinline__ h8 unpack_q4(uint32_t x) {
  const uint32_t M = 0x000F000Fu, E = 0x64006400u;
  h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  h2 a = __builtin_bit_cast(h2, (x & M) | E) + off;
  h2 b = __builtin_bit_cast(h2, ((x >> 4) & M) | E) + off;
  h2 c = __builtin_bit_cast(h2, ((x >> 8) & M) | E) + off;
  h2 d = __builtin_bit_cast(h2, ((x >> 12) & M) | E) + off;
  h8 r = {a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  return r;
}

__device__ __forceinline__ h8 unpack_q8(uint32_t x0, uint32_t x1) {
  const uint32_t M = 0x00FF00FFu, E = 0x64006400u;
  h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  uint32_t y0 = x0 ^ 0x80808080u, y1 = x1 ^ 0x80808080u;
  h2 a = __builtin_bit_cast(h2, (y0 & M) | E) + off;
  h2 b = __builtin_bit_cast(h2, ((y0 >> 8) & M) | E) + off;
  h2 c = __builtin_bit_cast(h2, (y1 & M) | E) + off;
  h2 d = __builtin_bit_cast(h2, ((y1 >> 8) & M) | E) + off;
  h8 r = {a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  return r;
}

// Workgroup: 4 waves.  With RH row halves the waves form CTW = 4/RH column
// tiles (16 columns each) x RH groups of RT row tiles.  Each wave owns its
// output tile over the workgroup's whole K range (64/S contiguous parts, a
// complete subtree of the canonical tree), so it accumulates parts in order and
// merges leaves with a binary-counter stack.  Activations are staged through a
// double-buffered LDS ring in chunks of 4 blocks and shared by all waves;
// weights stream as one 128-bit load per lane per chunk.  With S > 1 the K
// subtrees land in S output slices that the consumer combines as
// (s0+s1) or ((s0+s1)+(s2+s3)).
// Merge leaf `v` into the stack: t1 = trailing ones of the leaf index is the
// number of completed left siblings.  Written as compile-time recursion so every
// stack index is a constant before register promotion.
template <int T, int RT, int LOGP>
__device__ __forceinline__ void push_rec(int t1, float (&st)[LOGP][RT][4], float (&v)[RT][4],
                                         float (&fin)[RT][4]) {
  if constexpr (T == LOGP) {
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) fin[i][r] = v[i][r];
  } else {
    if (t1 == T) {
#pragma unroll
      for (int i = 0; i < RT; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) st[T][i][r] = v[i][r];
    } else {
#pragma unroll
      for (int i = 0; i < RT; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) v[i][r] = st[T][i][r] + v[i][r];
      push_rec<T + 1, RT, LOGP>(t1, st, v, fin);
    }
  }
}

template <int RT, int LOGP>
__device__ __forceinline__ void push_leaf_dyn(int leaf, float (&st)[LOGP][RT][4], float (&v)[RT][4],
                                              float (&fin)[RT][4]) {
  push_rec<0, RT, LOGP>(__builtin_ctz(~(unsigned)leaf), st, v, fin);
}

constexpr int QG_MT = 8;   // row tiles staged per workgroup (128 rows)

template <int RT, int RH, int BITS, int LOGP>
__global__ __launch_bounds__(256, 2) void k_qgemm(const uint32_t* __restrict__ W,
                                                  const uint16_t* __restrict__ Ws,
                                                  const _Float16* __restrict__ X,
                                                  const float* __restrict__ Xs, int nb, int mpad,
                                                  float* __restrict__ Y, int ldy, int m_rows,
                                                  size_t slice_stride) {
  constexpr int CTW = 4 / RH;
  constexpr int DW = BITS == 4 ? 1 : 2;
  constexpr int PPW = 1 << LOGP;
  __shared__ u32x4 s_act[2][QG_MT * 4 * 64];     // [buf][rt][bb][64 x 16B]
  __shared__ float s_xs[2][4][QG_MT * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nn = lane & 15, g = lane >> 4;
  const int ctw = wave % CTW, rh = wave / CTW;
  const int ct = blockIdx.x * CTW + ctw;
  const int q = blockIdx.y;
  const int rg = blockIdx.z;                       // group of QG_MT row tiles
  const int mt_all = mpad >> 4;
  const int mt = min(QG_MT, mt_all - rg * QG_MT);  // row tiles in this group
  const int nb4 = nb >> 2;
  const int c = (nb + 63) >> 6;
  const int p0 = q * PPW;
  const int b_begin = min(nb, p0 * c), b_end = min(nb, (p0 + PPW) * c);
  const int nchunk = (b_end - b_begin) >> 2;
  const uint32_t* Wt = W + (size_t)ct * nb4 * 256 * DW;
  const uint16_t* St = Ws + (size_t)ct * nb4 * 64;
  const u32x4* Xg = reinterpret_cast<const u32x4*>(X) + (size_t)rg * QG_MT * nb * 64;
  const int pieces = mt * 256;                     // 16-byte act pieces per chunk
  const int row0 = rg * QG_MT * 16;

  float st[LOGP][RT][4];
  float acc[RT][4], fin[RT][4];
#pragma unroll
  for (int i = 0; i < RT; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) { acc[i][r] = 0.0f; fin[i][r] = 0.0f; }

  // register staging for the next chunk (macros, so every array index is a
  // compile-time constant and stays in registers)
  u32x4 pa[QG_MT];
  float pxs[2];
  u32x4 pw[DW];
  u32x2 psc;
#define QG_LOAD_CHUNK(CH)                                                                        \
  do {                                                                                           \
    const int b0_ = b_begin + 4 * (CH), bq_ = b0_ >> 2;                                          \
    _Pragma("unroll") for (int k = 0; k < QG_MT; k++) {                                          \
      const int piece = min(tid + 256 * k, pieces - 1);                                          \
      pa[k] = Xg[((size_t)(piece >> 8) * nb + b0_) * 64 + (piece & 255)];                         \
    }                                                                                            \
    _Pragma("unroll") for (int k = 0; k < 2; k++) {                                              \
      const int e = tid + 256 * k;                                                               \
      const int rr = e & 127;                                                                    \
      const float v_ = Xs[(size_t)(b0_ + (e >> 7)) * mpad + row0 + min(rr, mt * 16 - 1)];         \
      pxs[k] = (rr < mt * 16) ? v_ : 0.0f;                                                       \
    }                                                                                            \
    const u32x4* wp_ = reinterpret_cast<const u32x4*>(Wt + ((size_t)bq_ * 256 + (g * 16 + nn) * 4) * DW); \
    _Pragma("unroll") for (int k = 0; k < DW; k++) pw[k] = wp_[k];                               \
    psc = *reinterpret_cast<const u32x2*>(St + ((size_t)bq_ * 16 + nn) * 4);                     \
  } while (0)
#define QG_STORE_CHUNK(BUF)                                                                      \
  do {                                                                                           \
    _Pragma("unroll") for (int k = 0; k < QG_MT; k++) s_act[(BUF)][tid + 256 * k] = pa[k];       \
    _Pragma("unroll") for (int k = 0; k < 2; k++) {                                              \
      const int e = tid + 256 * k;                                                               \
      s_xs[(BUF)][e >> 7][e & 127] = pxs[k];                                                     \
    }                                                                                            \
  } while (0)

  int leaf = 0;  // next leaf (part) index relative to p0
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  if (nchunk > 0) {
    QG_LOAD_CHUNK(0);
    QG_STORE_CHUNK(0);
  }
  __syncthreads();
  for (int ch = 0; ch < nchunk; ch++) {
    const int buf = ch & 1;
    u32x4 cw[DW];
#pragma unroll
    for (int k = 0; k < DW; k++) cw[k] = pw[k];
    const u32x2 csc = psc;
    if (ch + 1 < nchunk) QG_LOAD_CHUNK(ch + 1);
    const int b0 = b_begin + 4 * ch;
#pragma unroll
    for (int bb = 0; bb < 4; bb++) {
      h8 wv;
      if (BITS == 4) {
        const uint32_t x = bb == 0 ? cw[0][0] : bb == 1 ? cw[0][1] : bb == 2 ? cw[0][2] : cw[0][3];
        wv = unpack_q4(x);
      } else {
        const u32x4 lo = cw[bb >> 1];
        const uint32_t x0 = (bb & 1) ? lo[2] : lo[0], x1 = (bb & 1) ? lo[3] : lo[1];
        wv = unpack_q8(x0, x1);
      }
      const uint32_t sh = (bb < 2) ? csc[0] : csc[1];
      const float dw = h2f_bits((uint16_t)((bb & 1) ? (sh >> 16) : (sh & 0xFFFFu)));
#pragma unroll
      for (int i = 0; i < RT; i++) {
        const int rt = rh * RT + i;
        if (rt < mt) {
          const u32x4 a4 = s_act[buf][(rt * 4 + bb) * 64 + g * 16 + nn];
          const h8 av = __builtin_bit_cast(h8, a4);
          const f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, wv, zero, 0, 0, 0);
          const f4 xs = *reinterpret_cast<const f4*>(&s_xs[buf][bb][rt * 16 + g * 4]);
#pragma unroll
          for (int r = 0; r < 4; r++) acc[i][r] = __builtin_fmaf(d[r], dw * xs[r], acc[i][r]);
        }
      }
      const int b = b0 + bb;
      if ((b + 1) % c == 0 || b + 1 == nb) {
        push_leaf_dyn<RT, LOGP>(leaf, st, acc, fin);
        leaf++;
#pragma unroll
        for (int i = 0; i < RT; i++)
#pragma unroll
          for (int r = 0; r < 4; r++) acc[i][r] = 0.0f;
      }
    }
    if (ch + 1 < nchunk) QG_STORE_CHUNK(buf ^ 1);
    __syncthreads();
  }
#undef QG_LOAD_CHUNK
#undef QG_STORE_CHUNK
  // empty trailing parts of the subtree
  for (; leaf < PPW; leaf++) {
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][r] = 0.0f;
    push_leaf_dyn<RT, LOGP>(leaf, st, acc, fin);
  }
  float* Yq = Y + (size_t)q * slice_stride;
  const int col = ct * 16 + nn;
#pragma unroll
  for (int i = 0; i < RT; i++) {
    const int rt = rh * RT + i;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = row0 + rt * 16 + g * 4 + r;
      if (rt < mt && m < m_rows) Yq[(size_t)m * ldy + col] = fin[i][r];
    }
  }
}

int qgemm_splits(int n, int mpad) {
  const int mt = mpad / 16;
  const int rh = mt > 4 ? 2 : 1;
  const int ctw = 4 / rh;
  const int wgs = (n / 16 + ctw - 1) / ctw * ((mt + QG_MT - 1) / QG_MT);
  if (wgs >= 512) return 1;
  if (wgs * 2 >= 512) return 2;
  return 4;
}

hipError_t launch_qgemm(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y,
                        int ldy, int splits, size_t slice_stride) {
  const int nb = w.k / 32;
  const int mt_all = x.mpad / 16;
  const int mt = mt_all < QG_MT ? mt_all : QG_MT;
  const int rh = mt > 4 ? 2 : 1;
  const int rt = rh == 2 ? 4 : (mt > 2 ? 4 : (mt > 1 ? 2 : 1));
  const int ctw = 4 / rh;
  if ((w.n / 16) % ctw) return hipErrorInvalidValue;
  dim3 grid(w.n / 16 / ctw, splits, (mt_all + QG_MT - 1) / QG_MT);
  const uint32_t* W = (const uint32_t*)w.w;
#define RSTR_QG(R, H, B, LP)                                                                       \
  hipLaunchKernelGGL((k_qgemm<R, H, B, LP>), grid, dim3(256), 0, st, W, w.s, x.q, x.s, nb, x.mpad, y, \
                     ldy, m_rows, slice_stride)
#define RSTR_QG_S(R, H, B)                                 \
  do {                                                     \
    if (splits == 1) RSTR_QG(R, H, B, 6);                  \
    else if (splits == 2) RSTR_QG(R, H, B, 5);             \
    else RSTR_QG(R, H, B, 4);                              \
  } while (0)
#define RSTR_QG_R(B)                                       \
  do {                                                     \
    if (rh == 2) RSTR_QG_S(4, 2, B);                       \
    else if (rt == 4) RSTR_QG_S(4, 1, B);                  \
    else if (rt == 2) RSTR_QG_S(2, 1, B);                  \
    else RSTR_QG_S(1, 1, B);                               \
  } while (0)
  if (splits != 1 && splits != 2 && splits != 4) return hipErrorInvalidValue;
  if (w.bits == 4) RSTR_QG_R(4);
  else RSTR_QG_R(8);
#undef RSTR_QG_R
#undef RSTR_QG_S
#undef RSTR_QG
  return hipGetLastError();
}

__device__ __forceinline__ f4 sl_load4(const Slices& s, size_t i) {
  const f4 a = *reinterpret_cast<const f4*>(s.p + i);
  if (s.n == 1) return a;
  const f4 b = *reinterpret_cast<const f4*>(s.p + s.stride + i);
  f4 r;
  if (s.n == 2) {
#pragma unroll
    for (int k = 0; k < 4; k++) r[k] = a[k] + b[k];
    return r;
  }
  const f4 c = *reinterpret_cast<const f4*>(s.p + 2 * s.stride + i);
  const f4 d = *reinterpret_cast<const f4*>(s.p + 3 * s.stride + i);
#pragma unroll
  for (int k = 0; k < 4; k++) r[k] = (a[k] + b[k]) + (c[k] + d[k]);
  return r;
}

// ===========================================================================
// Row kernels: one wavefront per row.  Canonical sum of squares: lane l owns
// float4 chunks c = l + 64i (elements 4c..4c+3), accumulates fmaf(x,x,acc) in
// element order, lanes combine by the pairwise tree.
// ===========================================================================
__device__ __forceinline__ float row_sumsq(const float* __restrict__ x, int n4, int lane) {
  float acc = 0.0f;
  for (int c = lane; c < n4; c += 64) {
    f4 v = *reinterpret_cast<const f4*>(x + 4 * c);
    acc = __builtin_fmaf(v[0], v[0], acc);
    acc = __builtin_fmaf(v[1], v[1], acc);
    acc = __builtin_fmaf(v[2], v[2], acc);
    acc = __builtin_fmaf(v[3], v[3], acc);
  }
  return wave_tree_sum(acc);
}

__device__ __forceinline__ float rms_scale(float ss, int n, float eps) {
  float mean = ss / (float)n;
  return 1.0f / __builtin_sqrtf(mean + eps);
}

// Quantise chunk c of row `row` (valid lanes only store) into the MFMA tile
// layout.  A 32-element block spans 8 consecutive lanes of one round.
__device__ __forceinline__ void quant_store(f4 y, bool valid, int c, int row, int nb, int mpad,
                                            _Float16* __restrict__ Q, float* __restrict__ S) {
  float a = valid ? fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3]))) : 0.0f;
  a = fmaxf(a, __shfl_xor(a, 1, 64));
  a = fmaxf(a, __shfl_xor(a, 2, 64));
  a = fmaxf(a, __shfl_xor(a, 4, 64));
  if (!valid) return;
  float d = a / 127.0f;
  float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  h4 q;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float v = __builtin_rintf(y[i] * id);
    v = fminf(127.0f, fmaxf(-127.0f, v));
    q[i] = (_Float16)v;
  }
  int b = c >> 3, g = (c & 7) >> 1, s0 = (c & 1) * 4;
  size_t off = ((((size_t)(row >> 4) * nb + b) * 4 + g) * 16 + (row & 15)) * 8 + s0;
  *reinterpret_cast<h4*>(Q + off) = q;
  if ((c & 7) == 0) S[(size_t)b * mpad + row] = d;
}

__global__ __launch_bounds__(256) void k_rms_quant(const float* __restrict__ x,
                                                   const float* __restrict__ g, float goff, float eps,
                                                   int rows, int n, _Float16* __restrict__ Q,
                                                   float* __restrict__ S, int mpad) {
  int lane = threadIdx.x & 63;
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + (size_t)row * n;
  int n4 = n >> 2, nb = n >> 5;
  float r = rms_scale(row_sumsq(xr, n4, lane), n, eps);
  for (int c0 = 0; c0 < n4; c0 += 64) {
    int c = c0 + lane;
    bool valid = c < n4;
    f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valid) {
      f4 v = *reinterpret_cast<const f4*>(xr + 4 * c);
      f4 gg = *reinterpret_cast<const f4*>(g + 4 * c);
#pragma unroll
      for (int i = 0; i < 4; i++) y[i] = (v[i] * r) * (goff + gg[i]);
    }
    quant_store(y, valid, c, row, nb, mpad, Q, S);
  }
}

hipError_t launch_rms_quant(hipStream_t st, const float* x, const float* g, float goff, float eps,
                            int rows, int n, ActBuf& out) {
  hipLaunchKernelGGL(k_rms_quant, dim3((rows + 3) / 4), dim3(256), 0, st, x, g, goff, eps, rows, n,
                     out.q, out.s, out.mpad);
  return hipGetLastError();
}

// xmid = x + (sandwich ? rms(o, paln) : o); then rms(xmid, pfln) -> quantised.
// (decoder_gpu.clj layer-form: post-attn norm, residual-add!, pre-ffn norm.)
// The same kernel serves the post-ffn step: xout = xmid + (rms(dn, pffln) | dn)
// followed by the next layer's input norm (or the final norm of the head).
__global__ __launch_bounds__(256) void k_residual_norm_quant(
    Slices o, const float* __restrict__ x, float* __restrict__ xout,
    const float* __restrict__ post, const float* __restrict__ gnext, float goff, float eps, int rows,
    int n, _Float16* __restrict__ Q, float* __restrict__ S, int mpad) {
  int lane = threadIdx.x & 63;
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  int n4 = n >> 2, nb = n >> 5;
  const size_t orow = (size_t)row * n;
  const float* xr = x + (size_t)row * n;
  float* xo = xout + (size_t)row * n;
  float r1 = 1.0f;
  if (post) {
    float a = 0.0f;
    for (int c = lane; c < n4; c += 64) {
      f4 v = sl_load4(o, orow + 4 * c);
      a = __builtin_fmaf(v[0], v[0], a);
      a = __builtin_fmaf(v[1], v[1], a);
      a = __builtin_fmaf(v[2], v[2], a);
      a = __builtin_fmaf(v[3], v[3], a);
    }
    r1 = rms_scale(wave_tree_sum(a), n, eps);
  }
  float acc = 0.0f;
  for (int c = lane; c < n4; c += 64) {
    f4 ov = sl_load4(o, orow + 4 * c);
    f4 xv = *reinterpret_cast<const f4*>(xr + 4 * c);
    if (post) {
      f4 pg = *reinterpret_cast<const f4*>(post + 4 * c);
#pragma unroll
      for (int i = 0; i < 4; i++) ov[i] = (ov[i] * r1) * (goff + pg[i]);
    }
    f4 xm;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      xm[i] = xv[i] + ov[i];
      acc = __builtin_fmaf(xm[i], xm[i], acc);
    }
    *reinterpret_cast<f4*>(xo + 4 * c) = xm;
  }
  float r2 = rms_scale(wave_tree_sum(acc), n, eps);
  for (int c0 = 0; c0 < n4; c0 += 64) {
    int c = c0 + lane;
    bool valid = c < n4;
    f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valid) {
      f4 v = *reinterpret_cast<const f4*>(xo + 4 * c);
      f4 gg = *reinterpret_cast<const f4*>(gnext + 4 * c);
#pragma unroll
      for (int i = 0; i < 4; i++) y[i] = (v[i] * r2) * (goff + gg[i]);
    }
    quant_store(y, valid, c, row, nb, mpad, Q, S);
  }
}

hipError_t launch_post_attn(hipStream_t st, Slices o, const float* x, float* xmid,
                            const float* paln, const float* pfln, float goff, float eps, int rows,
                            int n, ActBuf& out) {
  hipLaunchKernelGGL(k_residual_norm_quant, dim3((rows + 3) / 4), dim3(256), 0, st, o, x, xmid, paln,
                     pfln, goff, eps, rows, n, out.q, out.s, out.mpad);
  return hipGetLastError();
}

hipError_t launch_post_ffn(hipStream_t st, Slices dn, const float* xmid, float* xout,
                           const float* pffln, const float* gnext, float goff, float eps, int rows,
                           int n, ActBuf& out) {
  hipLaunchKernelGGL(k_residual_norm_quant, dim3((rows + 3) / 4), dim3(256), 0, st, dn, xmid, xout,
                     pffln, gnext, goff, eps, rows, n, out.q, out.s, out.mpad);
  return hipGetLastError();
}

// hh = act(gate) * up (gelu-mul! / silu-mul!), quantised for the down projection.
__global__ __launch_bounds__(256) void k_act_quant(Slices gu, int rows, int ff,
                                                   int geglu, _Float16* __restrict__ Q,
                                                   float* __restrict__ S, int mpad) {
  int lane = threadIdx.x & 63;
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t gr = (size_t)row * 2 * ff;
  int n4 = ff >> 2, nb = ff >> 5;
  for (int c0 = 0; c0 < n4; c0 += 64) {
    int c = c0 + lane;
    bool valid = c < n4;
    f4 y = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valid) {
      f4 gv = sl_load4(gu, gr + 4 * c);
      f4 uv = sl_load4(gu, gr + ff + 4 * c);
#pragma unroll
      for (int i = 0; i < 4; i++) y[i] = (geglu ? dgelu(gv[i]) : dsilu(gv[i])) * uv[i];
    }
    quant_store(y, valid, c, row, nb, mpad, Q, S);
  }
}

hipError_t launch_act_quant(hipStream_t st, Slices gu, int rows, int ff, int geglu,
                            ActBuf& out) {
  hipLaunchKernelGGL(k_act_quant, dim3((rows + 3) / 4), dim3(256), 0, st, gu, rows, ff, geglu, out.q,
                     out.s, out.mpad);
  return hipGetLastError();
}

// Per (row, head): optional per-head RMSNorm (qk-norm), RoPE at positions[row]
// (HF rotate-half: y_i = x_i c - x_{i+h} s, y_{i+h} = x_{i+h} c + x_i s),
// then q -> qr (f32), k -> fp16 page slot, v -> fp16 page slot (slot -1 skips).
// (decoder_gpu.clj layer-form steps qk-norm, rope-pos-rows-buf!, and the
// routed append of paged_append.clj:179-228.)
__global__ __launch_bounds__(64) void k_qkv_post(Slices y, int n_q, int n_kv,
                                                 int hd, const float* __restrict__ qn,
                                                 const float* __restrict__ kn, float goff, float eps,
                                                 const float* __restrict__ cos_t,
                                                 const float* __restrict__ sin_t,
                                                 const int32_t* __restrict__ positions,
                                                 const int32_t* __restrict__ slots,
                                                 float* __restrict__ qr, uint16_t* __restrict__ kp,
                                                 uint16_t* __restrict__ vp) {
  __shared__ float sh[256];
  int nh = n_q + 2 * n_kv;
  int row = blockIdx.x / nh, hh = blockIdx.x % nh;
  int lane = threadIdx.x;
  int qd = n_q * hd, kvr = n_kv * hd, ncols = qd + 2 * kvr;
  const size_t yr = (size_t)row * ncols;
  int slot = slots[row];
  int hd4 = hd >> 2;
  if (hh >= n_q + n_kv) {
    if (slot < 0) return;
    int j = hh - n_q - n_kv;
    const size_t src = yr + qd + kvr + j * hd;
    uint16_t* dst = vp + (size_t)slot * kvr + j * hd;
    for (int c = lane; c < hd4; c += 64) {
      f4 v = sl_load4(y, src + 4 * c);
#pragma unroll
      for (int i = 0; i < 4; i++) dst[4 * c + i] = f2h_bits(v[i]);
    }
    return;
  }
  bool is_q = hh < n_q;
  if (!is_q && slot < 0) return;
  const size_t src = is_q ? yr + hh * hd : yr + qd + (hh - n_q) * hd;
  const float* gn = is_q ? qn : kn;
  float r = 1.0f;
  if (gn) {
    float a = 0.0f;
    for (int c = lane; c < hd4; c += 64) {
      f4 v = sl_load4(y, src + 4 * c);
      a = __builtin_fmaf(v[0], v[0], a);
      a = __builtin_fmaf(v[1], v[1], a);
      a = __builtin_fmaf(v[2], v[2], a);
      a = __builtin_fmaf(v[3], v[3], a);
    }
    r = rms_scale(wave_tree_sum(a), hd, eps);
  }
  for (int c = lane; c < hd4; c += 64) {
    f4 v = sl_load4(y, src + 4 * c);
    if (gn) {
      f4 gg = *reinterpret_cast<const f4*>(gn + 4 * c);
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = (v[i] * r) * (goff + gg[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) sh[4 * c + i] = v[i];
  }
  __syncthreads();
  int half = hd >> 1;
  int pos = positions[row];
  const float* ct = cos_t + (size_t)pos * half;
  const float* stt = sin_t + (size_t)pos * half;
  for (int i = lane; i < half; i += 64) {
    float a = sh[i], b = sh[i + half], c = ct[i], s = stt[i];
    float o1 = (a * c) - (b * s);
    float o2 = (b * c) + (a * s);
    if (is_q) {
      float* dst = qr + ((size_t)row * n_q + hh) * hd;
      dst[i] = o1;
      dst[i + half] = o2;
    } else {
      uint16_t* dst = kp + (size_t)slot * kvr + (hh - n_q) * hd;
      dst[i] = f2h_bits(o1);
      dst[i + half] = f2h_bits(o2);
    }
  }
}

hipError_t launch_qkv_post(hipStream_t st, Slices yqkv, int rows, int n_q, int n_kv, int hd,
                           const float* qn, const float* kn, float goff, float eps,
                           const float* cos_t, const float* sin_t, const int32_t* positions,
                           const int32_t* slots, float* qr, uint16_t* kpages, uint16_t* vpages) {
  int nh = n_q + 2 * n_kv;
  hipLaunchKernelGGL(k_qkv_post, dim3(rows * nh), dim3(64), 0, st, yqkv, n_q, n_kv, hd, qn, kn, goff,
                     eps, cos_t, sin_t, positions, slots, qr, kpages, vpages);
  return hipGetLastError();
}

// ===========================================================================
// Ragged paged attention decode (paged_attention.clj:196-228).
// Work item = (lane, kv head, history split of `split` tokens); items are
// packed by a device-side lane table so ragged lanes cost only their pages.
// ===========================================================================
__global__ void k_attn_prep(int batch, int split, int window, int n_kv,
                            const int32_t* __restrict__ lengths, int32_t* __restrict__ tab) {
  // tab: lo[B] k0[B] nsplit[B] base[B+1]
  if (threadIdx.x != 0) return;
  int32_t* lo = tab;
  int32_t* k0 = tab + batch;
  int32_t* ns = tab + 2 * batch;
  int32_t* base = tab + 3 * batch;
  int32_t acc = 0;
  for (int b = 0; b < batch; b++) {
    int len = lengths[b];
    int l0 = 0, kk0 = 0, n = 0;
    if (len > 0) {
      l0 = window > 0 ? max(0, len - window) : 0;
      kk0 = l0 / split;
      n = (len - 1) / split - kk0 + 1;
    }
    lo[b] = l0;
    k0[b] = kk0;
    ns[b] = n;
    base[b] = acc;
    acc += n * n_kv;
  }
  base[batch] = acc;
}

hipError_t launch_attn_prep(hipStream_t st, const AttnGeom& g, const int32_t* lengths,
                            int32_t* lane_tab) {
  hipLaunchKernelGGL(k_attn_prep, dim3(1), dim3(64), 0, st, g.batch, g.split, g.window, g.n_kv,
                     lengths, lane_tab);
  return hipGetLastError();
}

// Canonical split partial.  QK: LPT lanes per token, lane j owns 8-dim chunks
// c = j + LPT*i whose slices are c mod 16; slices merge by the fixed tree
// (bit 3, 2, 1, 0 of the slice index), the last levels across lanes.
// Softmax: m = max, p = exp(s - m).  PV: lane group g (16 lanes) takes tokens
// t = g mod 4 in order, lanes own contiguous dims; groups merge ((0+1)+(2+3)).
template <int HD, int G, int LPT>
__global__ __launch_bounds__(64) void k_attn_split(
    int batch, int n_kv, int page_size, int pps, int split, float scale,
    const float* __restrict__ q, const uint16_t* __restrict__ kp, const uint16_t* __restrict__ vp,
    const int32_t* __restrict__ page_table, const int32_t* __restrict__ lengths,
    const int32_t* __restrict__ tab, float* __restrict__ part) {
  constexpr int NCH = HD / 8;            // 8-dim chunks per head
  constexpr int NCL = NCH / LPT;         // chunks per lane
  constexpr int NSL = 16 / LPT;          // slice slots per lane (LPT <= 16)
  constexpr int TPR = 64 / LPT;          // tokens per QK round
  constexpr int DPL = HD / 16;           // PV dims per lane
  extern __shared__ float sc[];          // [G][split]
  const int lane = threadIdx.x;
  const int32_t* lo_t = tab;
  const int32_t* k0_t = tab + batch;
  const int32_t* ns_t = tab + 2 * batch;
  const int32_t* base = tab + 3 * batch;
  const int total = base[batch];
  const int kvr = n_kv * HD;
  const int ts = lane / LPT, j = lane % LPT;
  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    // lane b: base[b] <= item < base[b+1]
    int lo = 0, hi = batch;
    while (hi - lo > 1) {
      int mid = (lo + hi) >> 1;
      if (base[mid] <= item) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int ns = ns_t[b];
    const int rel = item - base[b];
    const int kvh = rel / ns;
    const int k = k0_t[b] + rel % ns;
    const int len = lengths[b];
    const int t0 = max(lo_t[b], k * split);
    const int t1 = min(len, (k + 1) * split);
    const int32_t* pt = page_table + (size_t)b * pps;
    // query slices for the G heads of this kv group
    float qv[G][NCL][8];
#pragma unroll
    for (int h = 0; h < G; h++) {
      const float* qh = q + ((size_t)b * (n_kv * G) + kvh * G + h) * HD;
#pragma unroll
      for (int i = 0; i < NCL; i++) {
        const int cch = j + LPT * i;
        f4 a = *reinterpret_cast<const f4*>(qh + 8 * cch);
        f4 bq = *reinterpret_cast<const f4*>(qh + 8 * cch + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) { qv[h][i][e] = a[e]; qv[h][i][4 + e] = bq[e]; }
      }
    }
    float mx[G];
#pragma unroll
    for (int h = 0; h < G; h++) mx[h] = -__builtin_inff();
    for (int T = t0 - (t0 % TPR); T < t1; T += TPR) {
      const int t = T + ts;
      const bool valid = (t >= t0) && (t < t1);
      float s[G][NSL];
#pragma unroll
      for (int h = 0; h < G; h++)
#pragma unroll
        for (int u = 0; u < NSL; u++) s[h][u] = 0.0f;
      if (valid) {
        const int page = pt[t / page_size];
        const uint16_t* krow = kp + ((size_t)page * page_size + (t % page_size)) * kvr + kvh * HD;
#pragma unroll
        for (int i = 0; i < NCL; i++) {
          const int cch = j + LPT * i;
          const h8 kv = *reinterpret_cast<const h8*>(krow + 8 * cch);
#pragma unroll
          for (int h = 0; h < G; h++)
#pragma unroll
            for (int e = 0; e < 8; e++)
              s[h][i % NSL] = __builtin_fmaf(qv[h][i][e], (float)kv[e], s[h][i % NSL]);
        }
      }
#pragma unroll
      for (int h = 0; h < G; h++) {
        float v;
        if constexpr (LPT == 4) v = (s[h][0] + s[h][2]) + (s[h][1] + s[h][3]);
        else if constexpr (LPT == 8) v = s[h][0] + s[h][1];
        else v = s[h][0];
#pragma unroll
        for (int m = LPT / 2; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, 64);
        const float score = v * scale;
        if (valid) {
          if (j == 0) sc[h * split + (t - t0)] = score;
          mx[h] = fmaxf(mx[h], score);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; h++) mx[h] = wave_max(mx[h]);
    __syncthreads();
    const int nt = t1 - t0;
    for (int i = lane; i < nt; i += 64)
#pragma unroll
      for (int h = 0; h < G; h++) sc[h * split + i] = dexp(sc[h * split + i] - mx[h]);
    __syncthreads();
    const int grp = lane >> 4, e16 = lane & 15;
    float o[G][DPL], l[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
      l[h] = 0.0f;
#pragma unroll
      for (int d = 0; d < DPL; d++) o[h][d] = 0.0f;
    }
    for (int T = t0 & ~3; T < t1; T += 4) {
      const int t = T + grp;
      if (t >= t0 && t < t1) {
        const int page = pt[t / page_size];
        const uint16_t* vrow =
            vp + ((size_t)page * page_size + (t % page_size)) * kvr + kvh * HD + e16 * DPL;
        float vv[DPL];
        if constexpr (DPL >= 8) {
#pragma unroll
          for (int d8 = 0; d8 < DPL; d8 += 8) {
            const h8 hv = *reinterpret_cast<const h8*>(vrow + d8);
#pragma unroll
            for (int e = 0; e < 8; e++) vv[d8 + e] = (float)hv[e];
          }
        } else {
          const h4 hv = *reinterpret_cast<const h4*>(vrow);
#pragma unroll
          for (int e = 0; e < 4; e++) vv[e] = (float)hv[e];
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
          const float p = sc[h * split + (t - t0)];
          l[h] = l[h] + p;
#pragma unroll
          for (int d = 0; d < DPL; d++) o[h][d] = __builtin_fmaf(p, vv[d], o[h][d]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
      l[h] = l[h] + __shfl_xor(l[h], 16, 64);
      l[h] = l[h] + __shfl_xor(l[h], 32, 64);
#pragma unroll
      for (int d = 0; d < DPL; d++) {
        o[h][d] = o[h][d] + __shfl_xor(o[h][d], 16, 64);
        o[h][d] = o[h][d] + __shfl_xor(o[h][d], 32, 64);
      }
    }
    float* pr = part + (size_t)item * G * (HD + 2);
    if (grp == 0) {
#pragma unroll
      for (int h = 0; h < G; h++) {
#pragma unroll
        for (int d = 0; d < DPL; d++) pr[h * (HD + 2) + e16 * DPL + d] = o[h][d];
        if (e16 == 0) {
          pr[h * (HD + 2) + HD] = mx[h];
          pr[h * (HD + 2) + HD + 1] = l[h];
        }
      }
    }
    __syncthreads();
  }
}

template <int HD, int G, int LPT>
static void launch_split_t(hipStream_t st, const AttnGeom& g, const float* q, const uint16_t* kp,
                           const uint16_t* vp, const int32_t* pt, const int32_t* len,
                           const int32_t* tab, float* part, int max_items) {
  int grid = max_items < 8192 ? max_items : 8192;
  if (grid < 1) grid = 1;
  size_t lds = sizeof(float) * G * g.split;
  hipLaunchKernelGGL((k_attn_split<HD, G, LPT>), dim3(grid), dim3(64), lds, st, g.batch, g.n_kv,
                     g.page_size, g.pps, g.split, g.scale, q, kp, vp, pt, len, tab, part);
}

hipError_t launch_attn_split(hipStream_t st, const AttnGeom& g, const float* q,
                             const uint16_t* kpages, const uint16_t* vpages,
                             const int32_t* page_table, const int32_t* lengths,
                             const int32_t* lane_tab, float* part, int max_items) {
  int G = g.n_q / g.n_kv;
#define RSTR_AS(HD_, G_, L_)                                                                   \
  if (g.hd == HD_ && G == G_) {                                                                \
    launch_split_t<HD_, G_, L_>(st, g, q, kpages, vpages, page_table, lengths, lane_tab, part, \
                                max_items);                                                    \
    return hipGetLastError();                                                                  \
  }
  RSTR_AS(64, 1, 4) RSTR_AS(64, 2, 4) RSTR_AS(64, 4, 4) RSTR_AS(64, 8, 4)
  RSTR_AS(128, 1, 4) RSTR_AS(128, 2, 4) RSTR_AS(128, 4, 4) RSTR_AS(128, 8, 8)
  RSTR_AS(256, 1, 4) RSTR_AS(256, 2, 8) RSTR_AS(256, 4, 8) RSTR_AS(256, 8, 16)
#undef RSTR_AS
  return hipErrorInvalidValue;
}

// Merge splits of one (lane, q head) in split order and quantise the row
// block for the output projection: w = exp(m_k - M), L = fmaf(l_k, w, L),
// O = fmaf(o_k, w, O), out = O / L.  Empty routes output 0.
template <int HD>
__global__ __launch_bounds__(64) void k_attn_merge(int batch, int n_q, int n_kv,
                                                   const int32_t* __restrict__ lengths,
                                                   const int32_t* __restrict__ tab,
                                                   const float* __restrict__ part,
                                                   float* __restrict__ out_f32,
                                                   _Float16* __restrict__ Q, float* __restrict__ S,
                                                   int mpad) {
  constexpr int DPL = HD / 64;
  const int lane = threadIdx.x;
  const int b = blockIdx.x / n_q, h = blockIdx.x % n_q;
  const int G = n_q / n_kv;
  const int ns = tab[2 * batch + b];
  const int base = tab[3 * batch + b] + (h / G) * ns;
  const int hl = h % G;
  const int len = lengths[b];
  float O[DPL];
#pragma unroll
  for (int d = 0; d < DPL; d++) O[d] = 0.0f;
  if (len > 0 && ns > 0) {
    const int stride = G * (HD + 2);
    float M = -__builtin_inff();
    for (int kk = lane; kk < ns; kk += 64)
      M = fmaxf(M, part[(size_t)(base + kk) * stride + hl * (HD + 2) + HD]);
    M = wave_max(M);
    float L = 0.0f;
    for (int kk = 0; kk < ns; kk++) {
      const float* pr = part + (size_t)(base + kk) * stride + hl * (HD + 2);
      const float w = dexp(pr[HD] - M);
      L = __builtin_fmaf(pr[HD + 1], w, L);
#pragma unroll
      for (int d = 0; d < DPL; d++) O[d] = __builtin_fmaf(pr[lane * DPL + d], w, O[d]);
    }
#pragma unroll
    for (int d = 0; d < DPL; d++) O[d] = O[d] / L;
  }
  if (out_f32) {
#pragma unroll
    for (int d = 0; d < DPL; d++) out_f32[((size_t)b * n_q + h) * HD + lane * DPL + d] = O[d];
  }
  if (Q) {
    // 32-dim blocks: 32/DPL lanes per block
    float a = 0.0f;
#pragma unroll
    for (int d = 0; d < DPL; d++) a = fmaxf(a, fabsf(O[d]));
#pragma unroll
    for (int m = 1; m < 32 / DPL; m <<= 1) a = fmaxf(a, __shfl_xor(a, m, 64));
    const float dq = a / 127.0f;
    const float id = (dq != 0.0f) ? 1.0f / dq : 0.0f;
    const int qd = n_q * HD, nb = qd >> 5;
#pragma unroll
    for (int d = 0; d < DPL; d++) {
      const int kcol = h * HD + lane * DPL + d;
      float v = __builtin_rintf(O[d] * id);
      v = fminf(127.0f, fmaxf(-127.0f, v));
      const int blk = kcol >> 5, g = (kcol & 31) >> 3, s = kcol & 7;
      Q[((((size_t)(b >> 4) * nb + blk) * 4 + g) * 16 + (b & 15)) * 8 + s] = (_Float16)v;
      if ((kcol & 31) == 0) S[(size_t)blk * mpad + b] = dq;
    }
  }
}

hipError_t launch_attn_merge(hipStream_t st, const AttnGeom& g, const int32_t* lengths,
                             const int32_t* lane_tab, const float* part, float* out_f32,
                             ActBuf* out_q) {
  dim3 grid(g.batch * g.n_q);
  _Float16* Q = out_q ? out_q->q : nullptr;
  float* S = out_q ? out_q->s : nullptr;
  int mpad = out_q ? out_q->mpad : 0;
  if (g.hd == 64)
    hipLaunchKernelGGL(k_attn_merge<64>, grid, dim3(64), 0, st, g.batch, g.n_q, g.n_kv, lengths,
                       lane_tab, part, out_f32, Q, S, mpad);
  else if (g.hd == 128)
    hipLaunchKernelGGL(k_attn_merge<128>, grid, dim3(64), 0, st, g.batch, g.n_q, g.n_kv, lengths,
                       lane_tab, part, out_f32, Q, S, mpad);
  else if (g.hd == 256)
    hipLaunchKernelGGL(k_attn_merge<256>, grid, dim3(64), 0, st, g.batch, g.n_q, g.n_kv, lengths,
                       lane_tab, part, out_f32, Q, S, mpad);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ===========================================================================
// Tail: argmax per row (ties -> lowest id, NaN beats finite, lowest NaN id)
// and embedding gather into the next resident input row (decode-tail!,
// decoder_gpu.clj:73-78).  Any reduction order gives the same winner.
// ===========================================================================
__device__ __forceinline__ bool arg_take(float av, int ai, float bv, int bi) {
  if (bi == INT_MAX) return false;
  if (ai == INT_MAX) return true;
  const bool an = av != av, bn = bv != bv;
  if (an) return bn && bi < ai;
  if (bn) return true;
  if (bv > av) return true;
  if (bv == av) return bi < ai;
  return false;
}

__global__ __launch_bounds__(1024) void k_argmax_gather(const float* __restrict__ logits, int vocab,
                                                        const float* __restrict__ emb, int d,
                                                        int32_t* __restrict__ tok,
                                                        float* __restrict__ r0) {
  __shared__ float sv[1024];
  __shared__ int si[1024];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* lr = logits + (size_t)row * vocab;
  float bv = 0.0f;
  int bi = INT_MAX;
  for (int i = tid; i < vocab; i += 1024) {
    const float v = lr[i];
    if (arg_take(bv, bi, v, i)) { bv = v; bi = i; }
  }
  sv[tid] = bv;
  si[tid] = bi;
  __syncthreads();
  for (int s = 512; s > 0; s >>= 1) {
    if (tid < s && arg_take(sv[tid], si[tid], sv[tid + s], si[tid + s])) {
      sv[tid] = sv[tid + s];
      si[tid] = si[tid + s];
    }
    __syncthreads();
  }
  const int t = si[0];
  if (tid == 0) tok[row] = t;
  const float* er = emb + (size_t)t * d;
  float* rr = r0 + (size_t)row * d;
  for (int i = tid; i < d; i += 1024) rr[i] = er[i];
}

hipError_t launch_argmax_gather(hipStream_t st, const float* logits, int rows, int vocab,
                                const float* emb, int d, int32_t* tok, float* r0) {
  hipLaunchKernelGGL(k_argmax_gather, dim3(rows), dim3(1024), 0, st, logits, vocab, emb, d, tok, r0);
  return hipGetLastError();
}

__global__ void k_gather_rows(const float* __restrict__ emb, int d, const int32_t* __restrict__ lanes,
                              const int32_t* __restrict__ tokens, float* __restrict__ r0) {
  const int i = blockIdx.x;
  const float* er = emb + (size_t)tokens[i] * d;
  float* rr = r0 + (size_t)lanes[i] * d;
  for (int k = threadIdx.x; k < d; k += blockDim.x) rr[k] = er[k];
}

hipError_t launch_gather_rows(hipStream_t st, const float* emb, int d, const int32_t* lanes,
                              const int32_t* tokens, int n, float* r0) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gather_rows, dim3(n), dim3(256), 0, st, emb, d, lanes, tokens, r0);
  return hipGetLastError();
}

// Routed paged append (doc/serving-architecture.md:178-190): f32 rows -> fp16
// round-to-nearest-even at slot = page*page_size + offset; slot -1 skips.
__global__ void k_append_rows(const float* __restrict__ k, const float* __restrict__ v, int kvr,
                              const int32_t* __restrict__ slots, uint16_t* __restrict__ kp,
                              uint16_t* __restrict__ vp) {
  const int row = blockIdx.x;
  const int slot = slots[row];
  if (slot < 0) return;
  for (int i = threadIdx.x; i < kvr; i += blockDim.x) {
    kp[(size_t)slot * kvr + i] = f2h_bits(k[(size_t)row * kvr + i]);
    vp[(size_t)slot * kvr + i] = f2h_bits(v[(size_t)row * kvr + i]);
  }
}

hipError_t launch_append_rows(hipStream_t st, const float* k_rows, const float* v_rows, int rows,
                              int kvr, const int32_t* slots, uint16_t* kpages, uint16_t* vpages) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_append_rows, dim3(rows), dim3(256), 0, st, k_rows, v_rows, kvr, slots, kpages,
                     vpages);
  return hipGetLastError();
}

// COW page copy: one physical page of every (slab, layer) (page_pool.clj:892-900).
__global__ void k_copy_pages(uint16_t* const* __restrict__ slabs, int nslabs, int64_t pe,
                             const int32_t* __restrict__ pairs) {
  const int pi = blockIdx.x / nslabs, s = blockIdx.x % nslabs;
  const int64_t src = (int64_t)pairs[2 * pi] * pe, dst = (int64_t)pairs[2 * pi + 1] * pe;
  uint16_t* base = slabs[s];
  const int64_t n8 = pe / 8;
  const uint4* sp = reinterpret_cast<const uint4*>(base + src);
  uint4* dp = reinterpret_cast<uint4*>(base + dst);
  for (int64_t i = threadIdx.x; i < n8; i += blockDim.x) dp[i] = sp[i];
}

hipError_t launch_copy_pages(hipStream_t st, uint16_t** slabs, int nslabs, int64_t page_elems,
                             const int32_t* pairs, int npairs) {
  if (npairs <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_copy_pages, dim3(npairs * nslabs), dim3(256), 0, st, slabs, nslabs, page_elems,
                     pairs);
  return hipGetLastError();
}

// Synthetic K/V, the stand-in for a restored prefix.  For each (layer, slab)
// RSTR_SYNTH_TEMPLATES page templates hold fp16(Irwin-Hall(12) N(0,1)) values
// keyed by (seed, layer, slab) and (template*page_elems + element); physical
// page p copies template (splitmix64(seed ^ p) >> 32) % RSTR_SYNTH_TEMPLATES.
// Filling is then a bandwidth-bound copy.
__global__ void k_gen_templates(uint16_t* __restrict__ tmpl, int n_layers, int64_t pe, uint64_t seed) {
  const int s = blockIdx.y;                       // slab index = slab*L + layer
  const int layer = s % n_layers, slab = s / n_layers;
  const uint64_t key = tensor_key(seed, layer, 64 + slab);
  const int64_t total = (int64_t)RSTR_SYNTH_TEMPLATES * pe;
  uint16_t* base = tmpl + (size_t)s * total;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x)
    base[i] = f2h_bits(synth_normal(key, (uint64_t)i, 0.0, 1.0));
}

hipError_t launch_gen_templates(hipStream_t st, uint16_t* tmpl, int n_layers, int64_t page_elems,
                                uint64_t seed) {
  hipLaunchKernelGGL(k_gen_templates, dim3(256, 2 * n_layers), dim3(256), 0, st, tmpl, n_layers,
                     page_elems, seed);
  return hipGetLastError();
}

__global__ void k_fill_synthetic(uint16_t* const* __restrict__ slabs, int nslabs, int64_t pe,
                                 const uint16_t* __restrict__ tmpl, const int32_t* __restrict__ pages,
                                 uint64_t seed) {
  const int pi = blockIdx.y;
  const int s = blockIdx.x;
  const int64_t page = pages[pi];
  const int t = (int)((splitmix64(seed ^ (uint64_t)page) >> 32) % RSTR_SYNTH_TEMPLATES);
  const uint4* src = reinterpret_cast<const uint4*>(tmpl + ((size_t)s * RSTR_SYNTH_TEMPLATES + t) * pe);
  uint4* dst = reinterpret_cast<uint4*>(slabs[s] + (size_t)page * pe);
  for (int64_t i = threadIdx.x; i < pe / 8; i += blockDim.x) dst[i] = src[i];
}

hipError_t launch_fill_synthetic(hipStream_t st, uint16_t** slabs, int n_layers,
                                 int64_t page_elems, const uint16_t* tmpl, const int32_t* pages,
                                 int npages, uint64_t seed) {
  if (npages <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_synthetic, dim3(2 * n_layers, npages), dim3(256), 0, st, slabs,
                     2 * n_layers, page_elems, tmpl, pages, seed);
  return hipGetLastError();
}

}  // namespace rstr

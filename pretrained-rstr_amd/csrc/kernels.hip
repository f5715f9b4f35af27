// kernels.hip -- gfx950 kernels of the resident continuous decode step.
//
// Each kernel reproduces one op of the reference decode step
// (src/pretrained/decoder_gpu.clj:122-220 layer/head order, :64-91 tail)
// with the canonical fp32 operation order documented next to it, so the CPU
// restatement can check every intermediate bit-for-bit.
#include "device_math.h"
#include "kernels.h"

#include <algorithm>
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
  S[((((size_t)ct * nb4 + bq) * 4 + (nn >> 2)) * 4 + bb) * 4 + (nn & 3)] = scale;
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
// Dequantising linear on MFMA: y[m][n] = sum_b (isum(m,n,b) * dx[m,b]) * dw[n,b]
// ===========================================================================
// The activation operand holds q_x*dx in fp16, exact because the activation
// scale has a 4-bit significand (act_scale).  v_mfma_f32_16x16x32_f16 then
// returns t = isum*dx exactly: every product q_w*(q_x*dx) is an integer times
// the power of two under dx's significand, and every partial sum stays below
// 2^24 of those units, so no addition rounds whatever the MFMA's order.
// Canonical block order: the nb blocks form 4 contiguous quarters; each
// quarter accumulates acc = fmaf(t, dw, acc) in block order from +0 (one
// v_fma_mix_f32 with the fp16 weight scale); y = (q0 + q1) + (q2 + q3).
//
// The MFMA takes the weights as the A operand and the activations as B, so a
// lane's accumulator holds 4 consecutive output columns (n = 4*(lane/16) + r)
// of one row (m = lane%16): it needs the 4 weight scales of its columns per
// block and column tile.

#define RSTR_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// A VGPR holding a constant the compiler cannot fold, so or(and(x, M), E)
// selects one v_and_or_b32 (M in an SGPR, E in this VGPR).
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(c));
  return r;
}

// Q4 dword (nibble i at bits 4i carries k_local {0,2,4,6,1,3,5,7}[i]) -> the
// 8 fp16 integers q - 8 in k order.  Even nibbles: (x & 0x000F000F) | 0x6400
// is the fp16 value 1024 + n; odd nibbles stay in bits 4..7, giving 1024 + 16n,
// which one exact packed fma maps to n - 8.  E = 0x64006400.
__device__ __forceinline__ h8 unpack_q4(uint32_t x, uint32_t E) {
  const uint32_t x8 = x >> 8;
  h2 a = __builtin_bit_cast(h2, (x & 0x000F000Fu) | E);
  h2 b = __builtin_bit_cast(h2, (x & 0x00F000F0u) | E);
  h2 c = __builtin_bit_cast(h2, (x8 & 0x000F000Fu) | E);
  h2 d = __builtin_bit_cast(h2, (x8 & 0x00F000F0u) | E);
  const h2 o1 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 o2 = {(_Float16)-72.0f, (_Float16)-72.0f};
  a = a + o1;
  b = __builtin_elementwise_fma(b, s16, o2);
  c = c + o1;
  d = __builtin_elementwise_fma(d, s16, o2);
  h8 r = {a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  return r;
}

// Q8 dword pair (byte i carries k_local {0,2,1,3,4,6,5,7}[i]) -> 8 fp16 q.
__device__ __forceinline__ h8 unpack_q8(uint32_t x0, uint32_t x1, uint32_t E) {
  const uint32_t y0 = x0 ^ 0x80808080u, y1 = x1 ^ 0x80808080u;
  const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  h2 a = __builtin_bit_cast(h2, (y0 & 0x00FF00FFu) | E) + off;
  h2 b = __builtin_bit_cast(h2, ((y0 >> 8) & 0x00FF00FFu) | E) + off;
  h2 c = __builtin_bit_cast(h2, (y1 & 0x00FF00FFu) | E) + off;
  h2 d = __builtin_bit_cast(h2, ((y1 >> 8) & 0x00FF00FFu) | E) + off;
  h8 r = {a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  return r;
}

// hh = act(gate) * up for the 8 consecutive inputs k0..k0+7 of row m of the
// down projection, from the gate/up slices added in the canonical tree (the
// arithmetic of k_act_quant); rows past m_rows give 0.
__device__ __forceinline__ void act_in_row8(const ActIn& a, int m, int m_rows, int k0, float hh[8]) {
  if (m >= m_rows) {
#pragma unroll
    for (int e = 0; e < 8; e++) hh[e] = 0.0f;
    return;
  }
  const size_t r = (size_t)m * 2 * a.ff + k0;
  f4 g[4][2], u[4][2];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int sk = k < a.S ? k : 0;
    const float* p = a.gu + sk * a.stride + r;
    g[k][0] = *reinterpret_cast<const f4*>(p);
    g[k][1] = *reinterpret_cast<const f4*>(p + 4);
    u[k][0] = *reinterpret_cast<const f4*>(p + a.ff);
    u[k][1] = *reinterpret_cast<const f4*>(p + a.ff + 4);
  }
#pragma unroll
  for (int h = 0; h < 2; h++) {
    f4 gv, uv;
    if (a.S == 1) { gv = g[0][h]; uv = u[0][h]; }
    else if (a.S == 2) {
#pragma unroll
      for (int i = 0; i < 4; i++) { gv[i] = g[0][h][i] + g[1][h][i]; uv[i] = u[0][h][i] + u[1][h][i]; }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        gv[i] = (g[0][h][i] + g[1][h][i]) + (g[2][h][i] + g[3][h][i]);
        uv[i] = (u[0][h][i] + u[1][h][i]) + (u[2][h][i] + u[3][h][i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) hh[4 * h + i] = (a.geglu ? dgelu(gv[i]) : dsilu(gv[i])) * uv[i];
  }
}

// |max| over the 8 values of one lane (the caller reduces across the lanes of
// the 32-block), then the quantised integers of a block scale d by the rule of
// quant_store: q = rint(hh / d) clamped to +-127.
__device__ __forceinline__ float amax8(const float hh[8]) {
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) a = fmaxf(a, fabsf(hh[e]));
  return a;
}
__device__ __forceinline__ void quant8(const float hh[8], float d, float q[8]) {
  const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) q[e] = fminf(127.0f, fmaxf(-127.0f, __builtin_rintf(hh[e] * id)));
}

// Workgroup: 4 waves over the same RT row tiles (RT*16 rows) and K range, wave
// w owning column tiles (4*blockIdx.x + w)*CT ..+CT-1.  The K range is NQ whole
// quarters (split s of 4/NQ); with NQ < 4 the workgroups of one column block
// write 4/NQ output slices that the consumer combines as (s0+s1) or
// ((s0+s1)+(s2+s3)).  A chunk is KC blocks (KC = 4, or 1 when a quarter is not
// a whole number of 4-block groups).  Activation fragments (RT*KC KB) reach a
// double-buffered LDS ring by direct-to-LDS DMA, shared by the 4 waves;
// weights and weight scales stream into registers one chunk ahead.  Row tiles past the batch compute on clamped rows and are never
// stored, which keeps the hot loop free of branches.
//
// ACT (gate/up with the gated activation fused, one K slice): workgroup x
// owns activation block x of the down projection's input, i.e. gate columns
// 32x..32x+31 (waves 0, 1) and the same up columns (waves 2, 3).  Every wave
// runs all four quarters, so y = (q0 + q1) + (q2 + q3) as the sliced path's
// consumer forms it; the epilogue stages y in LDS and writes
// act(gate) * up quantised (the rule of k_act_quant) into `ep`, and the fp32
// gate/up output is never written.
struct ActEpi {
  _Float16* q;   // quantised activations of the down projection (MFMA tile order)
  float* s;      // block scales [nb_out][mpad]
  int mpad, nb_out, geglu;
};

// QB (one K slice, quarters of qs = nb/4 blocks that are not whole 4-block
// chunks, e.g. K = 640): chunks stay 4-block groups and a quarter ends at
// whichever block of a chunk closes it, so the loads stay 16 bytes per lane
// and the chain order is unchanged.
//
// PL > 0 (at most PL chunks: short K slices such as K = 640 in four slices, or
// 16-row tiles over 4..8 chunks of 4 blocks): every chunk's weights, scales and
// activation DMA are issued at once and the chain runs after one wait, instead
// of one dependent memory round trip per chunk.
template <int RT, int CT, int BITS, int NQ, int KC, bool NT, bool ACT = false, bool QB = false, int PL = 0>
__global__ __launch_bounds__(256, ACT ? 4 : 2) void k_qgemm(const uint32_t* __restrict__ W,
                                                const uint16_t* __restrict__ Ws,
                                                const _Float16* __restrict__ X,
                                                const float* __restrict__ Xs, int nb, int nct,
                                                int mpad, float* __restrict__ Y, int ldy,
                                                int m_rows, size_t slice_stride, ActEpi ep) {
  static_assert(!ACT || (RT == 4 && CT == 1 && NQ == 4), "fused activation: 64x16 wave tiles, one K slice");
  static_assert(!QB || (NQ == 4 && KC == 4 && !ACT), "quarters inside chunks: one K slice, 4-block chunks");
  static_assert(PL == 0 || (!ACT && !QB && (KC == 1 || RT == 1)), "preloaded chains: 1-block chunks or 16-row tiles");
  constexpr int DW = BITS == 4 ? 1 : 2;
  constexpr int ACT_KB = RT * KC;                  // 1 KB activation fragments per chunk
  constexpr int BUF_U4 = ACT_KB * 64;              // u32x4 units per ring buffer
  constexpr int AI = (ACT_KB + 3) / 4;             // activation DMAs per wave
  constexpr int EPI_U4 = ACT ? RT * 256 : 0;       // epilogue tile: 4 waves x RT*16 rows x 16 floats
  constexpr int NBUF = PL > 2 ? PL : 2;            // ring buffers (one per chunk when preloading)
  __shared__ u32x4 ring[NBUF * BUF_U4 > EPI_U4 ? NBUF * BUF_U4 : EPI_U4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nn = lane & 15, g = lane >> 4;
  const int ct0 = ACT ? (wave >> 1) * (nct >> 1) + 2 * (int)blockIdx.x + (wave & 1) : (blockIdx.x * 4 + wave) * CT;
  const int split = blockIdx.y;
  const int rg = blockIdx.z;
  const int row0 = rg * RT * 16;
  const int mt = min(RT, (mpad >> 4) - rg * RT);
  const int nb4 = nb >> 2, qs = nb >> 2;
  const int cpq = qs / KC;
  const int nchunk = QB ? nb / KC : NQ * cpq;
  const int b_begin = split * NQ * qs;
  const uint32_t E = opaque_vgpr(0x64006400u);

  // per-lane DMA sources and weight offsets (chunk-invariant parts)
  const _Float16* xsrc[AI];  // wave-uniform bases; each lane adds lane*16 bytes
#pragma unroll
  for (int i = 0; i < AI; i++) {
    const int a = min(wave + 4 * i, ACT_KB - 1);
    const int rt = min(a / KC, mt - 1), kc = a % KC;
    xsrc[i] = X + ((size_t)(rg * RT + rt) * nb + b_begin + kc) * 512;
  }
  const uint32_t* wsrc[CT];  // wave-uniform
  const uint32_t* ssrc[CT];
#pragma unroll
  for (int c = 0; c < CT; c++) {
    const int ctl = min(ct0 + c, nct - 1);
    const int bq0 = b_begin >> 2;
    wsrc[c] = W + ((size_t)ctl * nb4 + bq0) * 256 * DW;
    ssrc[c] = reinterpret_cast<const uint32_t*>(Ws + ((size_t)ctl * nb4 + bq0) * 64);
  }
  const int wlane = (g * 16 + nn) * 4 * DW;  // dwords
  const int slane = g * 8;                   // dwords

  auto issue_dma = [&](int ch, int buf) {
    u32x4* base = ring + buf * BUF_U4;
#pragma unroll
    for (int i = 0; i < AI; i++) {
      const int a = wave + 4 * i;
      if (ACT_KB % 4 == 0 || a < ACT_KB)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(xsrc[i] + (size_t)ch * KC * 512 + lane * 8),
                                         RSTR_LDS_PTR(base + a * 64), 16, 0, 0);
    }
  };

  // weights and scales: streamed past L2 when this launch reads each weight
  // once (one row group), cached when a second row group re-reads them
  auto ld_w = [](const auto* p) { if constexpr (NT) return ld_stream(p); else return *p; };
  auto load_w = [&](int ch, uint32_t (&pw)[CT][KC * DW], uint32_t (&psc)[CT][KC * 2]) {
    const int b = ch * KC;  // relative to b_begin
#pragma unroll
    for (int c = 0; c < CT; c++) {
      if constexpr (KC == 4) {
        const uint32_t* wp = wsrc[c] + (size_t)(b >> 2) * 256 * DW + wlane;
        const uint32_t* sp = ssrc[c] + (size_t)(b >> 2) * 32 + slane;
        const u32x4 w0 = ld_w(reinterpret_cast<const u32x4*>(wp));
#pragma unroll
        for (int k = 0; k < 4; k++) pw[c][k] = w0[k];
        if constexpr (DW == 2) {
          const u32x4 w1 = ld_w(reinterpret_cast<const u32x4*>(wp + 4));
#pragma unroll
          for (int k = 0; k < 4; k++) pw[c][4 + k] = w1[k];
        }
        const u32x4 s0 = ld_w(reinterpret_cast<const u32x4*>(sp));
        const u32x4 s1 = ld_w(reinterpret_cast<const u32x4*>(sp + 4));
#pragma unroll
        for (int k = 0; k < 4; k++) { psc[c][k] = s0[k]; psc[c][4 + k] = s1[k]; }
      } else if constexpr (KC == 2) {
        // two blocks of one 4-block group (quarters of an even block count)
        const int ba = b_begin + b;
        const int bq = (ba >> 2) - (b_begin >> 2), bb = ba & 3;
        const uint32_t* wp = wsrc[c] + (size_t)bq * 256 * DW + wlane;
        const uint32_t* sp = ssrc[c] + (size_t)bq * 32 + slane;
        if constexpr (DW == 1) {
          const u32x2 w = ld_w(reinterpret_cast<const u32x2*>(wp + bb));
          pw[c][0] = w[0];
          pw[c][1] = w[1];
        } else {
          const u32x4 w = ld_w(reinterpret_cast<const u32x4*>(wp + 2 * bb));
#pragma unroll
          for (int k = 0; k < 4; k++) pw[c][k] = w[k];
        }
        const u32x4 s = ld_w(reinterpret_cast<const u32x4*>(sp + 2 * bb));
#pragma unroll
        for (int k = 0; k < 4; k++) psc[c][k] = s[k];
      } else {
        const int ba = b_begin + b;
        const int bq = (ba >> 2) - (b_begin >> 2), bb = ba & 3;
        const uint32_t* wp = wsrc[c] + (size_t)bq * 256 * DW + wlane;
        const uint32_t* sp = ssrc[c] + (size_t)bq * 32 + slane;
        if constexpr (DW == 1) pw[c][0] = ld_w(wp + bb);
        else {
          const u32x2 w = ld_w(reinterpret_cast<const u32x2*>(wp + 2 * bb));
          pw[c][0] = w[0];
          pw[c][1] = w[1];
        }
        const u32x2 s = ld_w(reinterpret_cast<const u32x2*>(sp + 2 * bb));
        psc[c][0] = s[0];
        psc[c][1] = s[1];
      }
    }
  };

  float acc[RT][CT][4];
  float sv0[NQ > 1 ? RT : 1][CT][4];
  float sv1[NQ > 2 ? RT : 1][CT][4];
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < RT; i++)
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][c][r] = 0.0f;

  // quarter kq complete: q0 -> sv0, sv0 + q1 -> sv0, q2 -> sv1 (the last
  // quarter stays in acc); y = (q0 + q1) + (q2 + q3)
  auto end_quarter = [&](int kq) {
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
      for (int c = 0; c < CT; c++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          if (kq == 0) sv0[i][c][r] = acc[i][c][r];
          else if (kq == 1) sv0[i][c][r] = sv0[i][c][r] + acc[i][c][r];
          else sv1[NQ > 2 ? i : 0][c][r] = acc[i][c][r];
          acc[i][c][r] = 0.0f;
        }
  };

  auto compute = [&](int ch, int buf, const uint32_t (&cw)[CT][KC * DW], const uint32_t (&csc)[CT][KC * 2]) {
    const u32x4* abuf = ring + buf * BUF_U4;
#pragma unroll
    for (int kc = 0; kc < KC; kc++) {
      h8 wv[CT];
      h2 dwh[CT][2];
#pragma unroll
      for (int c = 0; c < CT; c++) {
        if constexpr (BITS == 4) wv[c] = unpack_q4(cw[c][kc], E);
        else wv[c] = unpack_q8(cw[c][2 * kc], cw[c][2 * kc + 1], E);
        dwh[c][0] = __builtin_bit_cast(h2, csc[c][2 * kc]);
        dwh[c][1] = __builtin_bit_cast(h2, csc[c][2 * kc + 1]);
      }
      // software pipeline: the MFMAs of row tile i+1 issue before the VALU
      // work that consumes the results of row tile i
      f4 dn[CT];
      {
        const h8 av = __builtin_bit_cast(h8, abuf[kc * 64 + lane]);
#pragma unroll
        for (int c = 0; c < CT; c++) dn[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[c], av, zero, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < RT; i++) {
        f4 d[CT];
#pragma unroll
        for (int c = 0; c < CT; c++) d[c] = dn[c];
        if (i + 1 < RT) {
          const h8 av = __builtin_bit_cast(h8, abuf[((i + 1) * KC + kc) * 64 + lane]);
#pragma unroll
          for (int c = 0; c < CT; c++) dn[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[c], av, zero, 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            acc[i][c][r] = __builtin_fmaf(d[c][r], (float)dwh[c][r >> 1][r & 1], acc[i][c][r]);
      }
      if constexpr (QB) {
        const int nb_done = ch * KC + kc + 1;  // blocks of the chain done (wave-uniform)
        if (nb_done % qs == 0 && nb_done < nb) end_quarter(nb_done / qs - 1);
      }
    }
  };

  auto chunk = [&](int ch, const uint32_t (&cw)[CT][KC * DW], const uint32_t (&csc)[CT][KC * 2],
                   uint32_t (&nw)[CT][KC * DW], uint32_t (&nsc)[CT][KC * 2]) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of chunk ch
    __syncthreads();                     // every wave's DMA of chunk ch has landed
    if (ch + 1 < nchunk) {
      load_w(ch + 1, nw, nsc);
      issue_dma(ch + 1, (ch + 1) & 1);
    }
    compute(ch, ch & 1, cw, csc);
    if constexpr (NQ > 1 && !QB) {
      if ((ch + 1) % cpq == 0) {
        const int kq = (ch + 1) / cpq - 1;
        if (kq < NQ - 1) end_quarter(kq);
      }
    }
  };

  if constexpr (PL > 0) {
    uint32_t pwa[PL][CT][KC * DW], psa[PL][CT][KC * 2];
#pragma unroll
    for (int c = 0; c < PL; c++)
      if (c < nchunk) {
        load_w(c, pwa[c], psa[c]);
        issue_dma(c, c);
      }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of every chunk
    __syncthreads();                     // every wave's DMAs have landed
#pragma unroll
    for (int c = 0; c < PL; c++)
      if (c < nchunk) {
        compute(c, c, pwa[c], psa[c]);
        if constexpr (NQ > 1) {
          if ((c + 1) % cpq == 0 && (c + 1) / cpq - 1 < NQ - 1) end_quarter((c + 1) / cpq - 1);
        }
      }
  } else {
    uint32_t pw0[CT][KC * DW], ps0[CT][KC * 2], pw1[CT][KC * DW], ps1[CT][KC * 2];
    load_w(0, pw0, ps0);
    issue_dma(0, 0);
    for (int ch = 0; ch < nchunk; ch += 2) {
      chunk(ch, pw0, ps0, pw1, ps1);
      if (ch + 1 < nchunk) chunk(ch + 1, pw1, ps1, pw0, ps0);
    }
  }
  if constexpr (ACT) {
    // y tile -> LDS [wave][row][16 columns], then one thread per (row, 8 columns)
    // of the 32-column block: hh = act(gate) * up, block amax over its 4 lanes,
    // quantised as quant_store does, one 16-byte store of q*d
    float* T = reinterpret_cast<float*>(ring);
    __syncthreads();  // every wave has finished reading the ring
#pragma unroll
    for (int i = 0; i < RT; i++) {
      f4 o;
#pragma unroll
      for (int r = 0; r < 4; r++) o[r] = sv0[i][0][r] + (sv1[i][0][r] + acc[i][0][r]);
      *reinterpret_cast<f4*>(T + ((wave * RT * 16 + i * 16 + nn) * 16 + 4 * g)) = o;
    }
    __syncthreads();
    const int r = tid >> 2, cg = tid & 3;  // row of the tile, 8-column group of the block
    const float* tg = T + (((cg >> 1) * RT * 16 + r) * 16 + 8 * (cg & 1));
    const float* tu = tg + 2 * RT * 16 * 16;
    const f4 g0 = *reinterpret_cast<const f4*>(tg), g1 = *reinterpret_cast<const f4*>(tg + 4);
    const f4 u0 = *reinterpret_cast<const f4*>(tu), u1 = *reinterpret_cast<const f4*>(tu + 4);
    float y[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      y[k] = (ep.geglu ? dgelu(g0[k]) : dsilu(g0[k])) * u0[k];
      y[4 + k] = (ep.geglu ? dgelu(g1[k]) : dsilu(g1[k])) * u1[k];
    }
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) a = fmaxf(a, fabsf(y[k]));
    a = fmaxf(a, xor_lane<1>(a));
    a = fmaxf(a, xor_lane<2>(a));
    const int m = row0 + r;
    if (m < m_rows) {
      const float d = act_scale(a);
      const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
      h8 q;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        float v = __builtin_rintf(y[k] * id);
        v = fminf(127.0f, fmaxf(-127.0f, v));
        q[k] = (_Float16)(v * d);  // exact: 7 + 4 significant bits
      }
      const int b = blockIdx.x;
      *reinterpret_cast<h8*>(ep.q + ((((size_t)(m >> 4) * ep.nb_out + b) * 4 + cg) * 16 + (m & 15)) * 8) = q;
      if (cg == 0) ep.s[(size_t)b * ep.mpad + m] = d;
    }
    return;
  }
  float* Yq = Y + (size_t)split * slice_stride;
#pragma unroll
  for (int i = 0; i < RT; i++) {
    const int m = row0 + i * 16 + nn;
    if (i >= mt || m >= m_rows) continue;
#pragma unroll
    for (int c = 0; c < CT; c++) {
      if (ct0 + c >= nct) continue;
      f4 o;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        if constexpr (NQ == 1) o[r] = acc[i][c][r];
        else if constexpr (NQ == 2) o[r] = sv0[i][c][r] + acc[i][c][r];
        else o[r] = sv0[i][c][r] + (sv1[i][c][r] + acc[i][c][r]);
      }
      *reinterpret_cast<f4*>(Yq + (size_t)m * ldy + (ct0 + c) * 16 + 4 * g) = o;
    }
  }
}


// ---- few-row projections: weight-streaming GEMV ------------------------------
// The same output slices as k_qgemm (split s of 4/NQ covers quarters
// s*NQ .. s*NQ+NQ-1, combined (q0+q1) or ((q0+q1)+(q2+q3)) inside a split)
// for M <= 4 rows, without the 16-row MFMA tile.  One wave per (column tile,
// split), three phases:
//  1. the split's activation rows are staged in LDS as int8 q = rint(x/d)
//     (x = q*d exactly, so this recovers q), byte-permuted to match the
//     nibble/byte order of the weight words, with sum(q) and d per block row;
//  2. weights stream: lane 4*nn + bb holds column nn and block bb of each
//     4-block group, so every weight load of the wave is 256 (Q4) or 512 (Q8)
//     contiguous bytes, GD groups in flight per lane, streamed past L2.  A Q4
//     word splits into two words of nibble bytes (two masks) and the block's
//     integer dot comes from v_dot4_i32_i8: isum = sum(n*q) - 8*sum(q) for
//     Q4 nibbles n = w + 8, sum(w*q) for Q8 bytes.  t = isum*d is exact in
//     fp32 (|isum| < 2^20 times a 4-bit significand), bit-equal to the MFMA
//     block dot; t and the weight scale go to LDS;
//  3. one lane per (column, row) runs the canonical chain
//     acc = fmaf(t_b, dw_b, acc) over the split's blocks in order.
__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)d << 24);
}

template <int M, int BITS, int NQ, int GD, int WV, bool AIN = false>
__global__ __launch_bounds__(64 * WV) void k_qgemv(const uint32_t* __restrict__ W, const uint16_t* __restrict__ Ws,
                                              const _Float16* __restrict__ X, const float* __restrict__ Xs,
                                              int nb, int mpad, float* __restrict__ Y, int ldy, int m_rows,
                                              size_t slice_stride, ActIn ain) {
  constexpr int DW = BITS == 4 ? 1 : 2;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nn = lane >> 2, bb = lane & 3;
  const int ct = blockIdx.x * WV + wave, split = blockIdx.y;
  const int nb4 = nb >> 2, qs = nb >> 2;
  const int b_begin = split * NQ * qs, nblk = NQ * qs, b_end = b_begin + nblk;
  const int bq_lo = b_begin >> 2, bq_hi = (b_end - 1) >> 2;
  const int npair = nblk * M;
  u32x4* xq = reinterpret_cast<u32x4*>(smem);                      // [pair][2] (8 words)
  int* xsum = reinterpret_cast<int*>(xq + 2 * npair);              // [pair]
  float* dsc = reinterpret_cast<float*>(xsum + npair);             // [pair]
  float* tt = dsc + npair + (size_t)wave * nblk * (M + 1) * 16;    // this wave's [block][M][16]
  float* dws = tt + (size_t)nblk * M * 16;                         // and [block][16]

  const uint32_t* wbase = W + (size_t)ct * nb4 * 256 * DW;
  const uint16_t* sbase = Ws + (size_t)ct * nb4 * 64 + (nn >> 2) * 16 + bb * 4 + (nn & 3);
  uint32_t wr[GD][4 * DW];
  uint16_t sr[GD];
  auto load = [&](int j, int bq) {
    bq = min(bq, bq_hi);
    const uint32_t* wp = wbase + (size_t)bq * 256 * DW;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      if constexpr (DW == 1) {
        wr[j][g] = ld_stream(wp + g * 64 + lane);
      } else {
        const u32x2 v = ld_stream(reinterpret_cast<const u32x2*>(wp + (g * 64 + lane) * 2));
        wr[j][2 * g] = v[0];
        wr[j][2 * g + 1] = v[1];
      }
    }
    sr[j] = ld_stream(sbase + (size_t)bq * 64);
  };
#pragma unroll
  for (int j = 0; j < GD; j++) load(j, bq_lo + j);

  // 1. activation rows -> int8 words; piece = (pair, k-group) per lane
  for (int p0 = 0; p0 < npair * 4; p0 += 64 * WV) {
    const int p = p0 + tid;
    const int pc = min(p, npair * 4 - 1);
    const int g = pc & 3, pr = pc >> 2, m = pr % M, b = b_begin + pr / M;
    int q[8], qsum = 0;
    float d;
    if constexpr (AIN) {
      // the gate's activation computed here: a quad of lanes holds one 32-block
      float hh[8], qf[8];
      act_in_row8(ain, m, m_rows, 32 * b + 8 * g, hh);
      float a = amax8(hh);
      a = fmaxf(a, xor_lane<1>(a));
      a = fmaxf(a, xor_lane<2>(a));
      d = act_scale(a);
      quant8(hh, d, qf);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        q[e] = (int)qf[e];
        qsum += q[e];
      }
    } else {
      const h8 xv = *reinterpret_cast<const h8*>(X + ((size_t)(b * 4 + g) * 16 + m) * 8);
      d = Xs[(size_t)b * mpad + m];
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        q[e] = (int)__builtin_rintf((float)xv[e] * id);
        qsum += q[e];
      }
    }
    qsum += __builtin_amdgcn_update_dpp(0, qsum, 0xB1, 0xF, 0xF, true);  // quad xor 1
    qsum += __builtin_amdgcn_update_dpp(0, qsum, 0x4E, 0xF, 0xF, true);  // quad xor 2
    if (p < npair * 4) {
      u32x2 wq;
      if constexpr (BITS == 4) {  // nibble bytes: k {0,4,1,5} and {2,6,3,7}
        wq[0] = pack_i8x4(q[0], q[4], q[1], q[5]);
        wq[1] = pack_i8x4(q[2], q[6], q[3], q[7]);
      } else {                    // Q8 bytes: k {0,2,1,3} and {4,6,5,7}
        wq[0] = pack_i8x4(q[0], q[2], q[1], q[3]);
        wq[1] = pack_i8x4(q[4], q[6], q[5], q[7]);
      }
      reinterpret_cast<u32x2*>(xq)[pr * 4 + g] = wq;
      if (g == 0) {
        xsum[pr] = qsum;
        dsc[pr] = d;
      }
    }
  }
  __syncthreads();

  // 2. stream the weights; block dots and scales into LDS
  for (int base = bq_lo; base <= bq_hi; base += GD) {
#pragma unroll
    for (int j = 0; j < GD; j++) {
      const int b = (base + j) * 4 + bb;
      const bool in = b >= b_begin && b < b_end;
      const int bl = min(max(b - b_begin, 0), nblk - 1);
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int g = 0; g < 4; g++) {
        if constexpr (BITS == 4) {
          lo[g] = wr[j][g] & 0x0F0F0F0Fu;
          hi[g] = (wr[j][g] >> 4) & 0x0F0F0F0Fu;
        } else {
          lo[g] = wr[j][2 * g];
          hi[g] = wr[j][2 * g + 1];
        }
      }
      const float dw = (float)__builtin_bit_cast(_Float16, sr[j]);
      load(j, base + j + GD);  // this slot's next group (clamped re-read past the end)
#pragma unroll
      for (int m = 0; m < M; m++) {
        const u32x4* xr = xq + (size_t)(bl * M + m) * 2;
        const u32x4 x0 = xr[0], x1 = xr[1];  // k-groups 0,1 and 2,3 (two words each)
        int raw = 0;
        raw = __builtin_amdgcn_sdot4((int)lo[0], (int)x0[0], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[0], (int)x0[1], raw, false);
        raw = __builtin_amdgcn_sdot4((int)lo[1], (int)x0[2], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[1], (int)x0[3], raw, false);
        raw = __builtin_amdgcn_sdot4((int)lo[2], (int)x1[0], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[2], (int)x1[1], raw, false);
        raw = __builtin_amdgcn_sdot4((int)lo[3], (int)x1[2], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[3], (int)x1[3], raw, false);
        const int isum = BITS == 4 ? raw - 8 * xsum[bl * M + m] : raw;
        if (in) tt[(bl * M + m) * 16 + nn] = (float)isum * dsc[bl * M + m];
      }
      if (in) dws[bl * 16 + nn] = dw;
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // the clamped re-reads past the end have returned
  __syncthreads();

  // 3. canonical chain, one lane per (column, row); unrolled 16 deep so that
  // many of the chain's LDS reads are in flight at once (one-row down
  // 4096 x 14336: 12.8 -> 12.2 us)
  if (lane < 16 * M) {
    const int c = lane & 15, m = lane >> 4;
    float part[NQ];
#pragma unroll
    for (int kq = 0; kq < NQ; kq++) {
      float acc = 0.0f;
      const int e0 = kq * qs;
#pragma unroll 16
      for (int bl = e0; bl < e0 + qs; bl++) acc = __builtin_fmaf(tt[(bl * M + m) * 16 + c], dws[bl * 16 + c], acc);
      part[kq] = acc;
    }
    float o;
    if constexpr (NQ == 1) o = part[0];
    else if constexpr (NQ == 2) o = part[0] + part[1];
    else o = (part[0] + part[1]) + (part[2] + part[3]);
    if (m < m_rows) Y[(size_t)split * slice_stride + (size_t)m * ldy + (size_t)ct * 16 + c] = o;
  }
}

// GEMV launch for m_rows <= 4 (rows of the first 16-row tile).  Returns
// hipErrorInvalidValue, before any device work, for a shape it does not serve.
namespace {
template <bool AIN_>
hipError_t qgemv_go(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy, int splits,
                    size_t slice_stride, const ActIn& ain) {
  const int nb = w.k / 32;
  if (m_rows < 1 || m_rows > 4 || w.n % 16 || nb % 4 || (splits != 1 && splits != 2 && splits != 4))
    return hipErrorInvalidValue;
  const int nq = 4 / splits, nblk = nq * (nb / 4);
  const int M = m_rows <= 1 ? 1 : m_rows <= 2 ? 2 : 4;
  const int nct = w.n / 16;
  const int WVN = (nct % 4 == 0 && (size_t)nblk * M * 40 + (size_t)nblk * 64 * (M + 1) * 4 <= 64 * 1024) ? 4 : 1;
  const size_t lds = (size_t)nblk * M * 40 + (size_t)nblk * 64 * (M + 1) * WVN;
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  const dim3 grid(nct / WVN, splits);
  const uint32_t* W = (const uint32_t*)w.w;
#define RSTR_GV(M_, B_, Q_)                                                                                  \
  do {                                                                                                       \
    if (WVN == 4)                                                                                            \
      hipLaunchKernelGGL((k_qgemv<M_, B_, Q_, 8, 4, AIN_>), grid, dim3(256), lds, st, W, w.s, x.q, x.s, nb, x.mpad, \
                         y, ldy, m_rows, slice_stride, ain);                                                 \
    else                                                                                                     \
      hipLaunchKernelGGL((k_qgemv<M_, B_, Q_, 8, 1, AIN_>), grid, dim3(64), lds, st, W, w.s, x.q, x.s, nb, x.mpad, \
                         y, ldy, m_rows, slice_stride, ain);                                                 \
  } while (0)
#define RSTR_GV_Q(M_, B_)                    \
  do {                                       \
    if (nq == 4) RSTR_GV(M_, B_, 4);         \
    else if (nq == 2) RSTR_GV(M_, B_, 2);    \
    else RSTR_GV(M_, B_, 1);                 \
  } while (0)
#define RSTR_GV_M(B_)                        \
  do {                                       \
    if (M == 1) RSTR_GV_Q(1, B_);            \
    else if (M == 2) RSTR_GV_Q(2, B_);       \
    else RSTR_GV_Q(4, B_);                   \
  } while (0)
  if (w.bits == 4) RSTR_GV_M(4);
  else if (w.bits == 8) RSTR_GV_M(8);
  else return hipErrorInvalidValue;
#undef RSTR_GV_M
#undef RSTR_GV_Q
#undef RSTR_GV
  return hipGetLastError();
}
}  // namespace

hipError_t launch_qgemv(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy,
                        int splits, size_t slice_stride) {
  return qgemv_go<false>(st, w, x, m_rows, y, ldy, splits, slice_stride, ActIn{});
}

// Workgroup form of the GEMV: one workgroup per (column tile, split) whose four
// waves take the split's 4-block groups round robin (wave w: groups w, w+4, ...),
// so up to 4*GD groups of one column tile are in flight at once; block dots and
// scales meet in LDS, and the quarter chains run one wave per quarter before
// wave 0 adds them in the canonical tree.  Same arithmetic as k_qgemv.
template <int M, int BITS, int NQ, int GD, bool AIN = false>
__global__ __launch_bounds__(256) void k_qgemv_wg(const uint32_t* __restrict__ W, const uint16_t* __restrict__ Ws,
                                                 const _Float16* __restrict__ X, const float* __restrict__ Xs,
                                                 int nb, int mpad, float* __restrict__ Y, int ldy, int m_rows,
                                                 size_t slice_stride, ActIn ain) {
  constexpr int DW = BITS == 4 ? 1 : 2;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nn = lane >> 2, bb = lane & 3;
  const int ct = blockIdx.x, split = blockIdx.y;
  const int nb4 = nb >> 2, qs = nb >> 2;
  const int b_begin = split * NQ * qs, nblk = NQ * qs, b_end = b_begin + nblk;
  const int bq_lo = b_begin >> 2, bq_hi = (b_end - 1) >> 2;
  const int npair = nblk * M;
  u32x4* xq = reinterpret_cast<u32x4*>(smem);                      // [pair][2] (8 words)
  int* xsum = reinterpret_cast<int*>(xq + 2 * npair);              // [pair]
  float* dsc = reinterpret_cast<float*>(xsum + npair);             // [pair]
  float* tt = dsc + npair;                                         // [block][M][16]
  float* dws = tt + (size_t)nblk * M * 16;                         // [block][16]
  float* pq = dws + (size_t)nblk * 16;                             // [quarter][M][16]

  const uint32_t* wbase = W + (size_t)ct * nb4 * 256 * DW;
  const uint16_t* sbase = Ws + (size_t)ct * nb4 * 64 + (nn >> 2) * 16 + bb * 4 + (nn & 3);
  uint32_t wr[GD][4 * DW];
  uint16_t sr[GD];
  auto load = [&](int j, int bq) {
    bq = min(bq, bq_hi);
    const uint32_t* wp = wbase + (size_t)bq * 256 * DW;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      if constexpr (DW == 1) {
        wr[j][g] = ld_stream(wp + g * 64 + lane);
      } else {
        const u32x2 v = ld_stream(reinterpret_cast<const u32x2*>(wp + (g * 64 + lane) * 2));
        wr[j][2 * g] = v[0];
        wr[j][2 * g + 1] = v[1];
      }
    }
    sr[j] = ld_stream(sbase + (size_t)bq * 64);
  };
#pragma unroll
  for (int j = 0; j < GD; j++) load(j, bq_lo + wave + 4 * j);

  // 1. activation rows -> int8 words (as k_qgemv)
  for (int p0 = 0; p0 < npair * 4; p0 += 256) {
    const int p = p0 + tid;
    const int pc = min(p, npair * 4 - 1);
    const int g = pc & 3, pr = pc >> 2, m = pr % M, b = b_begin + pr / M;
    int q[8], qsum = 0;
    float d;
    if constexpr (AIN) {
      // the gate's activation computed here: a quad of lanes holds one 32-block
      float hh[8], qf[8];
      act_in_row8(ain, m, m_rows, 32 * b + 8 * g, hh);
      float a = amax8(hh);
      a = fmaxf(a, xor_lane<1>(a));
      a = fmaxf(a, xor_lane<2>(a));
      d = act_scale(a);
      quant8(hh, d, qf);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        q[e] = (int)qf[e];
        qsum += q[e];
      }
    } else {
      const h8 xv = *reinterpret_cast<const h8*>(X + ((size_t)(b * 4 + g) * 16 + m) * 8);
      d = Xs[(size_t)b * mpad + m];
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        q[e] = (int)__builtin_rintf((float)xv[e] * id);
        qsum += q[e];
      }
    }
    qsum += __builtin_amdgcn_update_dpp(0, qsum, 0xB1, 0xF, 0xF, true);  // quad xor 1
    qsum += __builtin_amdgcn_update_dpp(0, qsum, 0x4E, 0xF, 0xF, true);  // quad xor 2
    if (p < npair * 4) {
      u32x2 wq;
      if constexpr (BITS == 4) {
        wq[0] = pack_i8x4(q[0], q[4], q[1], q[5]);
        wq[1] = pack_i8x4(q[2], q[6], q[3], q[7]);
      } else {
        wq[0] = pack_i8x4(q[0], q[2], q[1], q[3]);
        wq[1] = pack_i8x4(q[4], q[6], q[5], q[7]);
      }
      reinterpret_cast<u32x2*>(xq)[pr * 4 + g] = wq;
      if (g == 0) {
        xsum[pr] = qsum;
        dsc[pr] = d;
      }
    }
  }
  __syncthreads();

  // 2. this wave's groups: block dots and scales into LDS
  for (int base = bq_lo + wave; base <= bq_hi; base += 4 * GD) {
#pragma unroll
    for (int j = 0; j < GD; j++) {
      const int bq = base + 4 * j;
      const int b = bq * 4 + bb;
      const bool in = b >= b_begin && b < b_end;  // false past bq_hi (clamped re-read)
      const int bl = min(max(b - b_begin, 0), nblk - 1);
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int g = 0; g < 4; g++) {
        if constexpr (BITS == 4) {
          lo[g] = wr[j][g] & 0x0F0F0F0Fu;
          hi[g] = (wr[j][g] >> 4) & 0x0F0F0F0Fu;
        } else {
          lo[g] = wr[j][2 * g];
          hi[g] = wr[j][2 * g + 1];
        }
      }
      const float dw = (float)__builtin_bit_cast(_Float16, sr[j]);
      if (base + 4 * GD <= bq_hi) load(j, bq + 4 * GD);
#pragma unroll
      for (int m = 0; m < M; m++) {
        const u32x4* xr = xq + (size_t)(bl * M + m) * 2;
        const u32x4 x0 = xr[0], x1 = xr[1];
        int raw = 0;
        raw = __builtin_amdgcn_sdot4((int)lo[0], (int)x0[0], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[0], (int)x0[1], raw, false);
        raw = __builtin_amdgcn_sdot4((int)lo[1], (int)x0[2], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[1], (int)x0[3], raw, false);
        raw = __builtin_amdgcn_sdot4((int)lo[2], (int)x1[0], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[2], (int)x1[1], raw, false);
        raw = __builtin_amdgcn_sdot4((int)lo[3], (int)x1[2], raw, false);
        raw = __builtin_amdgcn_sdot4((int)hi[3], (int)x1[3], raw, false);
        const int isum = BITS == 4 ? raw - 8 * xsum[bl * M + m] : raw;
        if (in) tt[(bl * M + m) * 16 + nn] = (float)isum * dsc[bl * M + m];
      }
      if (in) dws[bl * 16 + nn] = dw;
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // loads of waves without groups have returned
  __syncthreads();

  // 3. canonical chains: wave kq runs quarter kq, wave 0 adds the quarters
  if (wave < NQ && lane < 16 * M) {
    const int c = lane & 15, m = lane >> 4;
    float acc = 0.0f;
    const int e0 = wave * qs;
#pragma unroll 16
    for (int bl = e0; bl < e0 + qs; bl++) acc = __builtin_fmaf(tt[(bl * M + m) * 16 + c], dws[bl * 16 + c], acc);
    pq[(wave * M + m) * 16 + c] = acc;
  }
  if constexpr (NQ > 1) __syncthreads();
  if (wave == 0 && lane < 16 * M) {
    const int c = lane & 15, m = lane >> 4;
    float o;
    if constexpr (NQ == 1) o = pq[m * 16 + c];
    else if constexpr (NQ == 2) o = pq[m * 16 + c] + pq[(M + m) * 16 + c];
    else o = (pq[m * 16 + c] + pq[(M + m) * 16 + c]) + (pq[(2 * M + m) * 16 + c] + pq[(3 * M + m) * 16 + c]);
    if (m < m_rows) Y[(size_t)split * slice_stride + (size_t)m * ldy + (size_t)ct * 16 + c] = o;
  }
}

namespace {
template <bool AIN_>
hipError_t qgemv_wg_go(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy, int splits,
                       size_t slice_stride, const ActIn& ain) {
  const int nb = w.k / 32;
  if (m_rows < 1 || m_rows > 4 || w.n % 16 || nb % 4 || (splits != 1 && splits != 2 && splits != 4))
    return hipErrorInvalidValue;
  const int nq = 4 / splits, nblk = nq * (nb / 4);
  const int M = m_rows <= 1 ? 1 : m_rows <= 2 ? 2 : 4;
  const size_t lds = (size_t)nblk * M * 40 + (size_t)nblk * 64 * (M + 1) + (size_t)nq * M * 64;
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  const int ngroups = nblk % 4 == 0 ? nblk / 4 : (nblk + 3) / 4 + 1;  // groups a split touches, at most
  const dim3 grid(w.n / 16, splits);
  const uint32_t* W = (const uint32_t*)w.w;
#define RSTR_GV(M_, B_, Q_)                                                                                   \
  do {                                                                                                        \
    if (ngroups <= 8)                                                                                         \
      hipLaunchKernelGGL((k_qgemv_wg<M_, B_, Q_, 2, AIN_>), grid, dim3(256), lds, st, W, w.s, x.q, x.s, nb, \
                         x.mpad, y, ldy, m_rows, slice_stride, ain);                                          \
    else                                                                                                      \
      hipLaunchKernelGGL((k_qgemv_wg<M_, B_, Q_, 8, AIN_>), grid, dim3(256), lds, st, W, w.s, x.q, x.s, nb, \
                         x.mpad, y, ldy, m_rows, slice_stride, ain);                                          \
  } while (0)
#define RSTR_GV_Q(M_, B_)                    \
  do {                                       \
    if (nq == 4) RSTR_GV(M_, B_, 4);         \
    else if (nq == 2) RSTR_GV(M_, B_, 2);    \
    else RSTR_GV(M_, B_, 1);                 \
  } while (0)
#define RSTR_GV_M(B_)                        \
  do {                                       \
    if (M == 1) RSTR_GV_Q(1, B_);            \
    else if (M == 2) RSTR_GV_Q(2, B_);       \
    else RSTR_GV_Q(4, B_);                   \
  } while (0)
  if (w.bits == 4) RSTR_GV_M(4);
  else if (w.bits == 8) RSTR_GV_M(8);
  else return hipErrorInvalidValue;
#undef RSTR_GV_M
#undef RSTR_GV_Q
#undef RSTR_GV
  return hipGetLastError();
}
}  // namespace

hipError_t launch_qgemv_wg(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy,
                           int splits, size_t slice_stride) {
  return qgemv_wg_go<false>(st, w, x, m_rows, y, ldy, splits, slice_stride, ActIn{});
}

namespace {
struct QgPlan {
  int rt, ct, nq;
};
// Tile plan from the padded batch (row tiles) and the requested number of K
// slices (4/nq).  Measured on MI355X at the decode shapes (N 4096..128256,
// K 4096/14336, weights streamed from HBM): 64-row x 16-column wave tiles
// above 48 rows, except 32 x 16 with four K slices at 49..96 rows (more
// workgroups: QKV, O and down 15-20% faster at 64 rows, 6-15% at 80 and 96;
// from 112 rows the 64-row tile is 2-4% faster again), 32 x 32 for 17..48
// rows; up to 16 rows, 16 x 16 per quarter (one K quarter per wave: the most
// waves streaming weights, 20-28% faster than 16 x 32 at 1 and 16 rows),
// 16 x 64 for one-slice heads.
// One-slice heads whose quarters are not whole 4-block chunks (K = 640: the
// Gemma-3-270M head) run 4-block chunks with in-chunk quarter ends (QB), 16 x 32
// per wave: 262144 x 640 at 16 rows 55 -> 26 us (Q4), 102 -> 45 us (Q8); at one
// row 53 -> 22.6 us (Q4), 89 -> 38 us (Q8), against 1-block chunks.
QgPlan qg_plan(int mpad, int splits, int bits, int nb) {
  const int mt_all = mpad / 16;
  QgPlan p{};
  p.nq = 4 / splits;
  if (p.nq == 1 && mt_all >= 4 && mt_all <= 6) { p.rt = 2; p.ct = 1; }
  else if (mt_all > 3) { p.rt = 4; p.ct = 1; }
  else if (mt_all > 1) { p.rt = 2; p.ct = 2; }
  else if (p.nq == 4 && (nb / 4) % 4 != 0) { p.rt = 1; p.ct = 2; }
  else { p.rt = 1; p.ct = p.nq == 1 ? 1 : (p.nq == 4 && bits == 4) ? 4 : 2; }
  return p;
}
}  // namespace

// K slices for a projection of width n at this batch: one slice where the
// output is large and read once (gate/up at small batches, the head), two for
// wide projections, four where few column blocks would leave CUs idle.
int qgemm_splits(int n, int mpad, int bits) {
  (void)bits;
  const int mt_all = mpad / 16;
  if (mt_all > 3) return n >= 16384 ? 2 : 4;
  return 4;
}

// Launch arguments of one projection and the chunking choices made for it.
struct QgLaunch {
  dim3 grid;
  hipStream_t st;
  const uint32_t* W;
  const uint16_t* Ws;
  const _Float16* X;
  const float* Xs;
  int nb, nct, mpad;
  float* y;
  int ldy, m_rows;
  size_t slice_stride;
  bool kc4, once, pre, pre4;
};

template <int R, int C, int B, int Q, int K, bool N, bool QB, int PL>
static void qg_go(const QgLaunch& a) {
  hipLaunchKernelGGL((k_qgemm<R, C, B, Q, K, N, false, QB, PL>), a.grid, dim3(256), 0, a.st, a.W, a.Ws, a.X, a.Xs,
                     a.nb, a.nct, a.mpad, a.y, a.ldy, a.m_rows, a.slice_stride, ActEpi{});
}

// Chunking: 4-block chunks where the quarters are whole chunks; one K slice
// with quarters inside chunks (QB); every chunk preloaded for 16 x 16 wave
// tiles over 4..8 chunks (pre4) and for short 1-block-chunk slices (pre);
// 1-block chunks otherwise.
template <int R, int C, int B, int Q>
static void qg_go_tile(const QgLaunch& a) {
  if constexpr (R == 1 && C == 1) {
    if (a.pre4) { a.once ? qg_go<R, C, B, Q, 4, true, false, 8>(a) : qg_go<R, C, B, Q, 4, false, false, 8>(a); return; }
  }
  if (a.kc4) { a.once ? qg_go<R, C, B, Q, 4, true, false, 0>(a) : qg_go<R, C, B, Q, 4, false, false, 0>(a); return; }
  if constexpr (Q == 4) {
    a.once ? qg_go<R, C, B, 4, 4, true, true, 0>(a) : qg_go<R, C, B, 4, 4, false, true, 0>(a);
  } else {
    if (a.pre) { a.once ? qg_go<R, C, B, Q, 1, true, false, 8>(a) : qg_go<R, C, B, Q, 1, false, false, 8>(a); return; }
    a.once ? qg_go<R, C, B, Q, 1, true, false, 0>(a) : qg_go<R, C, B, Q, 1, false, false, 0>(a);
  }
}

template <int R, int C, int B>
static void qg_dispatch_q(const QgLaunch& a, int nq) {
  if (nq == 4) qg_go_tile<R, C, B, 4>(a);
  else if (nq == 2) qg_go_tile<R, C, B, 2>(a);
  else qg_go_tile<R, C, B, 1>(a);
}

template <int B>
static void qg_dispatch_t(const QgLaunch& a, const QgPlan& p) {
  if (p.rt == 4) qg_dispatch_q<4, 1, B>(a, p.nq);
  else if (p.rt == 2 && p.ct == 1) qg_go_tile<2, 1, B, 1>(a);
  else if (p.rt == 2) qg_dispatch_q<2, 2, B>(a, p.nq);
  else if (p.ct == 4) qg_dispatch_q<1, 4, B>(a, p.nq);
  else if (p.ct == 2) qg_dispatch_q<1, 2, B>(a, p.nq);
  else qg_dispatch_q<1, 1, B>(a, p.nq);
}

hipError_t launch_qgemm_form(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy,
                             int splits, size_t slice_stride, int form) {
  const int nb = w.k / 32;
  if (w.n % 16 || nb % 4 || (splits != 1 && splits != 2 && splits != 4)) return hipErrorInvalidValue;
  if (w.bits != 4 && w.bits != 8) return hipErrorInvalidValue;
  if (form == QG_FORM_WAVE_GEMV) return launch_qgemv(st, w, x, m_rows, y, ldy, splits, slice_stride);
  if (form == QG_FORM_WG_GEMV) return launch_qgemv_wg(st, w, x, m_rows, y, ldy, splits, slice_stride);
  if (form != QG_FORM_AUTO && form != QG_FORM_TILE) return hipErrorInvalidValue;
  // Few rows: the weight-streaming GEMVs.  Measured on MI355X (weights streamed
  // from HBM, four K slices; us for the GEMV forms against the 16-row MFMA
  // tile): one row against a long K (the MLP down projection, 4096 x 14336)
  // takes k_qgemv, 12.8 us (13.6 for the workgroup form, 19.0 for the tile);
  // other shapes at one or two rows take the workgroup form k_qgemv_wg --
  // Llama-3-8B qkv 6.4 vs 7.1, o 5.5 vs 5.8, gate/up 15.6 vs 16.0 (Q8: 7.9 vs
  // 9.1, 6.5 vs 8.2, 23.7 vs 26.7), down at two rows 14.9 vs 19.8, Qwen3-0.6B
  // down 3.7 vs 4.7, Gemma-3-270M down 3.3 vs 4.0; at three and four rows the
  // tile wins on the 4096-wide shapes (o 6.7 vs 5.8) and the workgroup form
  // only on matrices up to 4M weights (Qwen3-0.6B down 4.3 vs 4.8).  Quarters
  // that are not whole 4-block groups (K = 640: Gemma-3-270M) stay on the tile,
  // whose preloaded chains were faster there (config1 0.750 vs 0.760 ms/step).
  if (form == QG_FORM_AUTO && x.mpad == 16 && m_rows <= 4) {
    if (m_rows == 1 && w.k >= 8192) {
      if (launch_qgemv(st, w, x, m_rows, y, ldy, splits, slice_stride) == hipSuccess) return hipSuccess;
    } else if (splits == 4 && (nb / 4) % 4 == 0 &&
               (m_rows <= 2 || (size_t)w.n * (size_t)w.k <= ((size_t)4 << 20))) {
      if (launch_qgemv_wg(st, w, x, m_rows, y, ldy, splits, slice_stride) == hipSuccess) return hipSuccess;
    } else if (splits == 1 && (nb / 4) % 4 == 0 && (m_rows == 1 || (m_rows == 2 && w.k <= 1024))) {
      // one-slice LM heads: Qwen3-0.6B 151936 x 1024 at one row 19.7 vs 26.7 us
      // (Q8 29.8 vs 36.5; two rows 22.3 vs 26.9), Llama-3-8B 128256 x 4096 Q8
      // 95 vs 108 (Q4 62.2 vs 61.7)
      if (launch_qgemv_wg(st, w, x, m_rows, y, ldy, splits, slice_stride) == hipSuccess) return hipSuccess;
    }
  }
  const QgPlan p = qg_plan(x.mpad, splits, w.bits, nb);
  const int nct = w.n / 16;
  const int mt_all = x.mpad / 16;
  const dim3 grid((nct + 4 * p.ct - 1) / (4 * p.ct), splits, (mt_all + p.rt - 1) / p.rt);
  const uint32_t* W = (const uint32_t*)w.w;
  const bool kc4 = (nb / 4) % 4 == 0;  // quarters are whole 4-block chunks
  const bool once = grid.z == 1;      // every weight is read by one workgroup
  // every chunk preloaded: 1-block chunks of short slices; Q4 16-row tiles over
  // 4..8 4-block chunks below 16384 columns (kernel benchmark, weights from HBM,
  // one and 16 rows: Llama-3-8B o 7.1 -> 5.7 us, qkv 7.3 -> 7.1; Qwen3 down 5.7 ->
  // 4.7; Gemma down 4.4 -> 4.0; slower at 2 chunks and for the 28672-wide gate/up;
  // Q8 doubles the preloaded registers and is left on the chunk loop)
  const int nchunk4 = (4 / splits) * (nb / 4) / 4;
  const bool pre = !kc4 && (4 / splits) * (nb / 4) <= 8;
  const bool pre4 = kc4 && p.rt == 1 && nchunk4 >= 4 && nchunk4 <= 8 && w.n < 16384 && w.bits == 4;
  QgLaunch L{grid, st, W, w.s, x.q, x.s, nb, nct, x.mpad, y, ldy, m_rows, slice_stride, kc4, once, pre, pre4};
  if (w.bits == 4) qg_dispatch_t<4>(L, p);
  else qg_dispatch_t<8>(L, p);
  return hipGetLastError();
}

hipError_t launch_qgemm(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, float* y, int ldy, int splits,
                        size_t slice_stride) {
  return launch_qgemm_form(st, w, x, m_rows, y, ldy, splits, slice_stride, QG_FORM_AUTO);
}

// Down projection at one to four rows with act(gate)*up computed while the
// GEMV stages its activations (the separate activation launch and its
// quantised buffer drop out of the step).  Served where launch_qgemm would run
// k_qgemv or k_qgemv_wg, with the same arithmetic; anything else returns
// hipErrorNotSupported before any device work, and the caller runs
// launch_act_quant + launch_qgemm instead.  Measured on MI355X: config1 (Gemma-3
// 270M, one lane) 0.737 -> 0.725 ms/step, the one-lane Llama-3-8B step unchanged
// (2.29 ms).  The same staging in the preloaded 16-row MFMA tile made config2
// slower (0.79 -> 0.98 ms/step): 40 workgroups each rebuilt a quarter of the
// activation for all 16 rows from four slices, so it is not used there.
hipError_t launch_qgemm_actin(hipStream_t st, const QTensor& w, const ActIn& ain, int mpad, int m_rows, float* y,
                              int ldy, int splits, size_t slice_stride) {
  const int nb = w.k / 32;
  if (mpad != 16 || m_rows < 1 || m_rows > 16 || w.k != ain.ff || !ain.gu || (ain.S != 1 && ain.S != 2 && ain.S != 4))
    return hipErrorNotSupported;
  if (w.n % 16 || nb % 4 || (splits != 1 && splits != 2 && splits != 4) || (w.bits != 4 && w.bits != 8))
    return hipErrorNotSupported;
  ActBuf x{};
  x.mpad = mpad;
  if (m_rows <= 4) {
    if (m_rows == 1 && w.k >= 8192) {
      if (qgemv_go<true>(st, w, x, m_rows, y, ldy, splits, slice_stride, ain) == hipSuccess) return hipSuccess;
    } else if (splits == 4 && (nb / 4) % 4 == 0 &&
               (m_rows <= 2 || (size_t)w.n * (size_t)w.k <= ((size_t)4 << 20))) {
      if (qgemv_wg_go<true>(st, w, x, m_rows, y, ldy, splits, slice_stride, ain) == hipSuccess) return hipSuccess;
    }
  }
  return hipErrorNotSupported;
}

// Gate/up with the gated activation fused (k_qgemm<4, 1, BITS, 4, KC, NT, true>):
// every workgroup covers all of K, so there are ff/32 workgroups per 64-row
// group, four resident per CU (128 VGPRs).  Used from 1536 workgroups on (1.5
// rounds of 256 CUs).  Measured on MI355X, Llama-3-8B shapes: at 512 rows
// (prefill tiles) the fused launch saves the 117 MB slice round trip of the
// separate activation kernel, 267 -> 262 ms per 4096-token prompt; at 128 rows
// (896 workgroups, less than one round) the two forms are equal within 0.3%.
bool qgemm_act_fused(int ff, int mpad) {
  const int mt_all = mpad / 16;
  if (ff % 32 || mt_all < 4) return false;
  return (size_t)(ff / 32) * ((mt_all + 3) / 4) >= 1536;
}

hipError_t launch_qgemm_act(hipStream_t st, const QTensor& w, const ActBuf& x, int m_rows, int ff, int geglu,
                            ActBuf& out) {
  const int nb = w.k / 32;
  if (w.n != 2 * ff || nb % 4 || !qgemm_act_fused(ff, x.mpad) || out.mpad != x.mpad) return hipErrorInvalidValue;
  if (w.bits != 4 && w.bits != 8) return hipErrorInvalidValue;
  const int nct = w.n / 16;
  const dim3 grid(ff / 32, 1, (x.mpad / 16 + 3) / 4);
  const uint32_t* W = (const uint32_t*)w.w;
  const bool kc4 = (nb / 4) % 4 == 0;
  const bool once = grid.z == 1;
  const ActEpi ep{out.q, out.s, out.mpad, ff / 32, geglu};
#define RSTR_QA_L(B, K, N)                                                                                   \
  hipLaunchKernelGGL((k_qgemm<4, 1, B, 4, K, N, true>), grid, dim3(256), 0, st, W, w.s, x.q, x.s, nb, nct, \
                     x.mpad, nullptr, 0, m_rows, 0, ep)
#define RSTR_QA(B)                                  \
  do {                                              \
    if (kc4 && once) RSTR_QA_L(B, 4, true);         \
    else if (kc4) RSTR_QA_L(B, 4, false);           \
    else if (once) RSTR_QA_L(B, 1, true);           \
    else RSTR_QA_L(B, 1, false);                    \
  } while (0)
  if (w.bits == 4) RSTR_QA(4);
  else RSTR_QA(8);
#undef RSTR_QA
#undef RSTR_QA_L
  return hipGetLastError();
}

// Slice sums in the canonical tree, (s0+s1) or ((s0+s1)+(s2+s3)), from loads
// issued together.
template <int S>
__device__ __forceinline__ f4 sl_comb(const f4 (&v)[S]) {
  if constexpr (S == 1) return v[0];
  f4 r;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    if constexpr (S == 2) r[k] = v[0][k] + v[1][k];
    else r[k] = (v[0][k] + v[1][k]) + (v[2][k] + v[3][k]);
  }
  return r;
}
template <int S>
__device__ __forceinline__ f4 sl_get(const Slices& s, size_t i) {
  f4 v[S];
#pragma unroll
  for (int k = 0; k < S; k++) v[k] = *reinterpret_cast<const f4*>(s.p + k * s.stride + i);
  return sl_comb<S>(v);
}

// ===========================================================================
// Row kernels: one 256-thread workgroup per row.  Canonical sum of squares:
// thread t owns float4 chunks c = t + 256i (elements 4c..4c+3, i.e. slot
// (element/4) mod 256), accumulates fmaf(x,x,acc) in element order; the 256
// slots combine by the pairwise tree (xor butterfly inside each wave, then
// ((w0+w1)+(w2+w3)) across the four waves).  A thread's CPT chunks are loaded
// together before any arithmetic, so a row costs one memory round trip per
// phase.
// ===========================================================================
__device__ __forceinline__ float block_tree_sum(float v, float* sh4) {
  v = wave_tree_sum(v);
  __syncthreads();  // sh4 may still be read by an earlier reduction
  if ((threadIdx.x & 63) == 0) sh4[threadIdx.x >> 6] = v;
  __syncthreads();
  return (sh4[0] + sh4[1]) + (sh4[2] + sh4[3]);
}

__device__ __forceinline__ float fma4_sq(f4 v, float acc) {
  acc = __builtin_fmaf(v[0], v[0], acc);
  acc = __builtin_fmaf(v[1], v[1], acc);
  acc = __builtin_fmaf(v[2], v[2], acc);
  return __builtin_fmaf(v[3], v[3], acc);
}

__device__ __forceinline__ float rms_scale(float ss, int n, float eps) {
  float mean = ss / (float)n;
  return 1.0f / __builtin_sqrtf(mean + eps);
}

// Quantise chunk c of row `row` (valid lanes only store) into the MFMA tile
// layout as fp16 q*d.  A 32-element block spans 8 consecutive lanes of one
// round.
__device__ __forceinline__ void quant_store(f4 y, bool valid, int c, int row, int nb, int mpad,
                                            _Float16* __restrict__ Q, float* __restrict__ S) {
  float a = valid ? fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3]))) : 0.0f;
  a = fmaxf(a, xor_lane<1>(a));
  a = fmaxf(a, xor_lane<2>(a));
  a = fmaxf(a, xor_lane<4>(a));
  if (!valid) return;
  const float d = act_scale(a);
  const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
  h4 q;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float v = __builtin_rintf(y[i] * id);
    v = fminf(127.0f, fmaxf(-127.0f, v));
    q[i] = (_Float16)(v * d);   // exact: 7 + 4 significant bits
  }
  int b = c >> 3, g = (c & 7) >> 1, s0 = (c & 1) * 4;
  size_t off = ((((size_t)(row >> 4) * nb + b) * 4 + g) * 16 + (row & 15)) * 8 + s0;
  *reinterpret_cast<h4*>(Q + off) = q;
  if ((c & 7) == 0) S[(size_t)b * mpad + row] = d;
}

template <int CPT>
__global__ __launch_bounds__(256) void k_rms_quant(const float* __restrict__ x,
                                                   const float* __restrict__ g, float goff, float eps,
                                                   int n, _Float16* __restrict__ Q,
                                                   float* __restrict__ S, int mpad) {
  __shared__ float sh4[4];
  const int tid = threadIdx.x, row = blockIdx.x;
  const float* xr = x + (size_t)row * n;
  const int n4 = n >> 2, nb = n >> 5;
  f4 xv[CPT], gg[CPT];
#pragma unroll
  for (int k = 0; k < CPT; k++) {
    const int cc = min(tid + 256 * k, n4 - 1);
    xv[k] = *reinterpret_cast<const f4*>(xr + 4 * cc);
    gg[k] = *reinterpret_cast<const f4*>(g + 4 * cc);
  }
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < CPT; k++)
    if (tid + 256 * k < n4) acc = fma4_sq(xv[k], acc);
  const float r = rms_scale(block_tree_sum(acc, sh4), n, eps);
#pragma unroll
  for (int k = 0; k < CPT; k++) {
    const int c = tid + 256 * k;
    f4 y;
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = (xv[k][i] * r) * (goff + gg[k][i]);
    quant_store(y, c < n4, c, row, nb, mpad, Q, S);
  }
}

#define RSTR_CPT_DISPATCH(N4, MACRO)          \
  do {                                        \
    const int cpt_ = ((N4) + 255) / 256;      \
    if (cpt_ <= 1) MACRO(1);                  \
    else if (cpt_ <= 2) MACRO(2);             \
    else if (cpt_ <= 4) MACRO(4);             \
    else if (cpt_ <= 8) MACRO(8);             \
    else if (cpt_ <= 16) MACRO(16);           \
    else return hipErrorInvalidValue;         \
  } while (0)

hipError_t launch_rms_quant(hipStream_t st, const float* x, const float* g, float goff, float eps,
                            int rows, int n, ActBuf& out) {
  if (rows <= 0) return hipSuccess;
#define RSTR_L(C) hipLaunchKernelGGL(k_rms_quant<C>, dim3(rows), dim3(256), 0, st, x, g, goff, eps, n, out.q, out.s, out.mpad)
  RSTR_CPT_DISPATCH(n / 4, RSTR_L);
#undef RSTR_L
  return hipGetLastError();
}

// xmid = x + (sandwich ? rms(o, paln) : o); then rms(xmid, pfln) -> quantised.
// (decoder_gpu.clj layer-form: post-attn norm, residual-add!, pre-ffn norm.)
// The same kernel serves the post-ffn step: xout = xmid + (rms(dn, pffln) | dn)
// followed by the next layer's input norm (or the final norm of the head).
template <int S, int CPT, bool POST>
__global__ __launch_bounds__(256) void k_residual_norm_quant(
    Slices o, const float* __restrict__ x, float* __restrict__ xout,
    const float* __restrict__ post, const float* __restrict__ gnext, float goff, float eps, int n,
    _Float16* __restrict__ Q, float* __restrict__ S_, int mpad) {
  __shared__ float sh4[4];
  const int tid = threadIdx.x, row = blockIdx.x;
  const int n4 = n >> 2, nb = n >> 5;
  const size_t orow = (size_t)row * n;
  f4 ov[CPT], xv[CPT], pg[POST ? CPT : 1], gg[CPT];
#pragma unroll
  for (int k = 0; k < CPT; k++) {
    const int cc = min(tid + 256 * k, n4 - 1);
    ov[k] = sl_get<S>(o, orow + 4 * cc);
    xv[k] = *reinterpret_cast<const f4*>(x + orow + 4 * cc);
    if constexpr (POST) pg[k] = *reinterpret_cast<const f4*>(post + 4 * cc);
    gg[k] = *reinterpret_cast<const f4*>(gnext + 4 * cc);
  }
  if constexpr (POST) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < CPT; k++)
      if (tid + 256 * k < n4) a = fma4_sq(ov[k], a);
    const float r1 = rms_scale(block_tree_sum(a, sh4), n, eps);
#pragma unroll
    for (int k = 0; k < CPT; k++)
#pragma unroll
      for (int i = 0; i < 4; i++) ov[k][i] = (ov[k][i] * r1) * (goff + pg[k][i]);
  }
  float acc = 0.0f;
  f4 xm[CPT];
#pragma unroll
  for (int k = 0; k < CPT; k++) {
    const int c = tid + 256 * k;
#pragma unroll
    for (int i = 0; i < 4; i++) xm[k][i] = xv[k][i] + ov[k][i];
    if (c < n4) {
      acc = fma4_sq(xm[k], acc);
      *reinterpret_cast<f4*>(xout + orow + 4 * c) = xm[k];
    }
  }
  const float r2 = rms_scale(block_tree_sum(acc, sh4), n, eps);
#pragma unroll
  for (int k = 0; k < CPT; k++) {
    const int c = tid + 256 * k;
    f4 y;
#pragma unroll
    for (int i = 0; i < 4; i++) y[i] = (xm[k][i] * r2) * (goff + gg[k][i]);
    quant_store(y, c < n4, c, row, nb, mpad, Q, S_);
  }
}

static hipError_t launch_residual_norm(hipStream_t st, Slices o, const float* x, float* xo,
                                       const float* post, const float* gnext, float goff, float eps,
                                       int rows, int n, ActBuf& out) {
  if (rows <= 0) return hipSuccess;
#define RSTR_L3(Sn, C, P)                                                                              \
  hipLaunchKernelGGL((k_residual_norm_quant<Sn, C, P>), dim3(rows), dim3(256), 0, st, o, x, xo, post, \
                     gnext, goff, eps, n, out.q, out.s, out.mpad)
#define RSTR_L2(C)                               \
  do {                                           \
    if (post) {                                  \
      if (o.n == 1) RSTR_L3(1, C, true);         \
      else if (o.n == 2) RSTR_L3(2, C, true);    \
      else RSTR_L3(4, C, true);                  \
    } else {                                     \
      if (o.n == 1) RSTR_L3(1, C, false);        \
      else if (o.n == 2) RSTR_L3(2, C, false);   \
      else RSTR_L3(4, C, false);                 \
    }                                            \
  } while (0)
  if (o.n != 1 && o.n != 2 && o.n != 4) return hipErrorInvalidValue;
  RSTR_CPT_DISPATCH(n / 4, RSTR_L2);
#undef RSTR_L2
#undef RSTR_L3
  return hipGetLastError();
}

hipError_t launch_post_attn(hipStream_t st, Slices o, const float* x, float* xmid,
                            const float* paln, const float* pfln, float goff, float eps, int rows,
                            int n, ActBuf& out) {
  return launch_residual_norm(st, o, x, xmid, paln, pfln, goff, eps, rows, n, out);
}

hipError_t launch_post_ffn(hipStream_t st, Slices dn, const float* xmid, float* xout,
                           const float* pffln, const float* gnext, float goff, float eps, int rows,
                           int n, ActBuf& out) {
  return launch_residual_norm(st, dn, xmid, xout, pffln, gnext, goff, eps, rows, n, out);
}

// hh = act(gate) * up (gelu-mul! / silu-mul!), quantised for the down projection.
// Element-wise with per-block quantisation: workgroups tile (row, 1024 columns).
template <int S>
__global__ __launch_bounds__(256) void k_act_quant(Slices gu, int ff, int geglu,
                                                   _Float16* __restrict__ Q,
                                                   float* __restrict__ Sc, int mpad) {
  const int row = blockIdx.y;
  const size_t gr = (size_t)row * 2 * ff;
  const int n4 = ff >> 2, nb = ff >> 5;
  const int c = blockIdx.x * 256 + threadIdx.x;
  const bool valid = c < n4;
  const int cc = valid ? c : n4 - 1;
  f4 gs[S], us[S];
#pragma unroll
  for (int k = 0; k < S; k++) {
    gs[k] = *reinterpret_cast<const f4*>(gu.p + k * gu.stride + gr + 4 * cc);
    us[k] = *reinterpret_cast<const f4*>(gu.p + k * gu.stride + gr + ff + 4 * cc);
  }
  const f4 gv = sl_comb<S>(gs), uv = sl_comb<S>(us);
  f4 y;
#pragma unroll
  for (int i = 0; i < 4; i++) y[i] = (geglu ? dgelu(gv[i]) : dsilu(gv[i])) * uv[i];
  quant_store(y, valid, c, row, nb, mpad, Q, Sc);
}

hipError_t launch_act_quant(hipStream_t st, Slices gu, int rows, int ff, int geglu,
                            ActBuf& out) {
  if (rows <= 0) return hipSuccess;
  dim3 grid((ff / 4 + 255) / 256, rows);
  if (gu.n == 1) hipLaunchKernelGGL(k_act_quant<1>, grid, dim3(256), 0, st, gu, ff, geglu, out.q, out.s, out.mpad);
  else if (gu.n == 2) hipLaunchKernelGGL(k_act_quant<2>, grid, dim3(256), 0, st, gu, ff, geglu, out.q, out.s, out.mpad);
  else if (gu.n == 4) hipLaunchKernelGGL(k_act_quant<4>, grid, dim3(256), 0, st, gu, ff, geglu, out.q, out.s, out.mpad);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// Per (row, head): optional per-head RMSNorm (qk-norm), RoPE at positions[row]
// (HF rotate-half: y_i = x_i c - x_{i+h} s, y_{i+h} = x_{i+h} c + x_i s),
// then q -> qr (f32), k -> fp16 page slot, v -> fp16 page slot (slot -1 skips).
// (decoder_gpu.clj layer-form steps qk-norm, rope-pos-rows-buf!, and the
// routed append of paged_append.clj:179-228.)  head_dim <= 256, so lane l
// holds chunk l (elements 4l..4l+3) of the head.
template <int S>
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
  const int nh = n_q + 2 * n_kv;
  const int row = blockIdx.x / nh, hh = blockIdx.x % nh;
  const int lane = threadIdx.x;
  const int qd = n_q * hd, kvr = n_kv * hd, ncols = qd + 2 * kvr;
  const size_t yr = (size_t)row * ncols;
  const int slot = slots[row];
  const int hd4 = hd >> 2;
  const bool have = lane < hd4;
  const int cc = have ? lane : 0;
  if (hh >= n_q + n_kv) {
    if (slot < 0) return;
    const int j = hh - n_q - n_kv;
    const f4 v = sl_get<S>(y, yr + qd + kvr + j * hd + 4 * cc);
    if (have) {
      uint16_t* dst = vp + (size_t)slot * kvr + j * hd;
#pragma unroll
      for (int i = 0; i < 4; i++) dst[4 * lane + i] = f2h_bits(v[i]);
    }
    return;
  }
  const bool is_q = hh < n_q;
  if (!is_q && slot < 0) return;
  const size_t src = is_q ? yr + hh * hd : yr + qd + (hh - n_q) * hd;
  const float* gn = is_q ? qn : kn;
  f4 v = sl_get<S>(y, src + 4 * cc);
  if (gn) {
    const f4 gg = *reinterpret_cast<const f4*>(gn + 4 * cc);
    float a = 0.0f;
    if (have) {
      a = __builtin_fmaf(v[0], v[0], a);
      a = __builtin_fmaf(v[1], v[1], a);
      a = __builtin_fmaf(v[2], v[2], a);
      a = __builtin_fmaf(v[3], v[3], a);
    }
    // head_dim/4 <= 64 chunks: lane l holds slot l alone, and the tree over
    // 64 lanes equals the 256-slot tree (the other slots are +0).
    const float r = rms_scale(wave_tree_sum(a), hd, eps);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = (v[i] * r) * (goff + gg[i]);
  }
  if (have) {
#pragma unroll
    for (int i = 0; i < 4; i++) sh[4 * lane + i] = v[i];
  }
  __syncthreads();
  const int half = hd >> 1;
  const int pos = positions[row];
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
  if (hd > 256 || hd % 4) return hipErrorInvalidValue;
  const int nh = n_q + 2 * n_kv;
#define RSTR_L(Sn)                                                                                       \
  hipLaunchKernelGGL(k_qkv_post<Sn>, dim3(rows * nh), dim3(64), 0, st, yqkv, n_q, n_kv, hd, qn, kn, goff, \
                     eps, cos_t, sin_t, positions, slots, qr, kpages, vpages)
  if (yqkv.n == 1) RSTR_L(1);
  else if (yqkv.n == 2) RSTR_L(2);
  else if (yqkv.n == 4) RSTR_L(4);
  else return hipErrorInvalidValue;
#undef RSTR_L
  return hipGetLastError();
}

// ===========================================================================
// Ragged paged attention decode (paged_attention.clj:196-228).
// Work item = (lane, kv head, history split of `split` tokens); items are
// packed by a device-side lane table so ragged lanes cost only their pages.
// ===========================================================================
// Per-lane item table.  Item (lane b, kv head h, split k) covers the visible
// tokens [max(lo, k*split), min(len, (k+1)*split)).  A split is full when it
// holds `split` tokens; only a lane's first (window start) and last split can
// be partial.
__global__ __launch_bounds__(1024) void k_attn_prep(int batch, int split, int window, int n_kv, int R,
                                                   int max_items, const int32_t* __restrict__ lengths,
                                                   int32_t* __restrict__ tab) {
  // tab: lo[B] k0[B] nsplit[B] base[B+1] fbase[B+1] pbase[B+1]; base, fbase
  // and pbase are exclusive prefix sums over lanes of the lane's items, full
  // items and partial items (integer sums: any order is exact)
  __shared__ int32_t s_a[1024], s_f[1024], s_p[1024], s_h[RSTR_NCH];
  int32_t* lo = tab;
  int32_t* k0 = tab + batch;
  int32_t* ns = tab + 2 * batch;
  int32_t* base = tab + 3 * batch;
  int32_t* fbase = tab + 4 * batch + 1;
  int32_t* pbase = tab + 5 * batch + 2;
  const int tid = threadIdx.x;
  int32_t carry_a = 0, carry_f = 0, carry_p = 0;
  for (int i = tid; i < RSTR_NCH; i += 1024) s_h[i] = 0;
  __syncthreads();
  for (int b0 = 0; b0 < batch; b0 += 1024) {
    const int b = b0 + tid;
    int l0 = 0, kk0 = 0, n = 0, f = 0;
    if (b < batch) {
      const int len = lengths[b];
      if (len > 0) {
        l0 = window > 0 ? max(0, len - window) : 0;
        kk0 = l0 / split;
        n = (len - 1) / split - kk0 + 1;
        const int f_t1 = min(len, (kk0 + 1) * split);
        const bool first_full = l0 == kk0 * split && f_t1 - l0 == split;
        const bool last_full = len % split == 0;
        f = n == 1 ? (first_full ? 1 : 0) : n - (first_full ? 0 : 1) - (last_full ? 0 : 1);
        // partial splits by chunk count (n_kv items each)
        if (!first_full) atomicAdd(&s_h[(f_t1 - (l0 & ~15) + 15) >> 4], n_kv);
        if (n > 1 && !last_full) {
          const int lt0 = (kk0 + n - 1) * split;
          atomicAdd(&s_h[(len - (lt0 & ~15) + 15) >> 4], n_kv);
        }
      }
      lo[b] = l0;
      k0[b] = kk0;
      ns[b] = n;
    }
    const int32_t va = b < batch ? n * n_kv : 0;
    const int32_t vf = b < batch ? f * n_kv : 0;
    const int32_t vp = va - vf;
    // inclusive Hillis-Steele scans over the 1024 lanes of this chunk
    s_a[tid] = va;
    s_f[tid] = vf;
    s_p[tid] = vp;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int32_t ta = tid >= off ? s_a[tid - off] : 0;
      const int32_t tf = tid >= off ? s_f[tid - off] : 0;
      const int32_t tp = tid >= off ? s_p[tid - off] : 0;
      __syncthreads();
      s_a[tid] += ta;
      s_f[tid] += tf;
      s_p[tid] += tp;
      __syncthreads();
    }
    if (b < batch) {
      base[b] = carry_a + s_a[tid] - va;
      fbase[b] = carry_f + s_f[tid] - vf;
      pbase[b] = carry_p + s_p[tid] - vp;
    }
    carry_a += s_a[1023];
    carry_f += s_f[1023];
    carry_p += s_p[1023];
    __syncthreads();
  }
  // More items than the work list holds (descriptors the host validation
  // rejects): the step gets no attention work, so every output is 0, instead
  // of items written past the list.  carry_a is the same in every thread.
  if (carry_a > max_items) {
    for (int b = tid; b < batch; b += 1024) {
      ns[b] = 0;
      base[b] = 0;
      fbase[b] = 0;
      pbase[b] = 0;
    }
    carry_a = carry_f = carry_p = 0;
    for (int i = tid; i < RSTR_NCH; i += 1024) s_h[i] = 0;
    __syncthreads();
  }
  // list offsets of the partial items by decreasing chunk count: boff[c] =
  // the partial items of all counts above c, an exclusive suffix sum over s_h
  // (inclusive scan over the reversed counts; thread r holds count NCH-1-r)
  static_assert(RSTR_NCH <= 1024, "one count per thread");
  const int32_t hv = tid < RSTR_NCH ? s_h[RSTR_NCH - 1 - tid] : 0;
  s_a[tid] = hv;
  __syncthreads();
  for (int off = 1; off < RSTR_NCH; off <<= 1) {
    const int32_t t = tid >= off ? s_a[tid - off] : 0;
    __syncthreads();
    s_a[tid] += t;
    __syncthreads();
  }
  if (tid < RSTR_NCH) {
    int32_t* boff = tab + attn_bucket_offset(batch);
    boff[RSTR_NCH - 1 - tid] = s_a[tid] - hv;
    boff[RSTR_NCH + (RSTR_NCH - 1 - tid)] = 0;  // fill cursor
  }
  if (tid == 0) {
    base[batch] = carry_a;
    fbase[batch] = carry_f;
    pbase[batch] = carry_p;
    // the split kernel's R waves take attn_static_rounds(N, R) static
    // rounds; the counter hands out the rest of the list
    const int arm = attn_static_rounds(carry_a, R) * R;
    tab[attn_ctl_offset(batch)] = arm;
    tab[attn_ctl_offset(batch) + 1] = arm;
  }
}

// The step's work list: every item once, full items first (in (lane, kv
// head, split) order), then the partial ones.  Wave w of the R resident waves
// takes list positions k*R + w for even rounds k and k*R + R-1-w for odd ones
// (a snake), so waves hold equal counts of full items and the partial ones
// even out the remainder.  Entry = (lane | kv head << 20, t0, t1, item index).
// Built once per step, read by every layer.
__global__ __launch_bounds__(256) void k_attn_items(int batch, int n_kv, int split,
                                                    const int32_t* __restrict__ lengths,
                                                    int32_t* __restrict__ tab,
                                                    int4* __restrict__ items) {
  const int32_t* lo_t = tab;
  const int32_t* k0_t = tab + batch;
  const int32_t* ns_t = tab + 2 * batch;
  const int32_t* base = tab + 3 * batch;
  const int32_t* fbase = tab + 4 * batch + 1;
  const int32_t* pbase = tab + 5 * batch + 2;
  // the lane prefix in LDS for the search below (a search through global
  // memory is a chain of dependent round trips)
  constexpr int SB = 2048;
  __shared__ int32_t s_base[SB];
  const bool lds = batch < SB;
  if (lds)
    for (int k = threadIdx.x; k <= batch; k += 256) s_base[k] = base[k];
  __syncthreads();
  const int32_t* sb = lds ? s_base : base;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= sb[batch]) return;
  // the last lane whose first item is <= i (lanes without items have
  // base[b] == base[b+1], so the search lands on the lane that holds i)
  int b = 0, hi = batch;
  while (hi - b > 1) {
    const int mid = (b + hi) >> 1;
    if (sb[mid] <= i) b = mid; else hi = mid;
  }
  const int ns = ns_t[b];
  const int rel = i - sb[b];
  const int kvh = rel / ns;
  const int s = rel % ns;
  const int len = lengths[b];
  const int k = k0_t[b] + s;
  const int t0 = max(lo_t[b], k * split), t1 = min(len, (k + 1) * split);
  const int nf = (fbase[b + 1] - fbase[b]) / n_kv;  // full splits of this lane
  const int l0 = lo_t[b];
  const bool first_partial = !(l0 == k0_t[b] * split && min(len, (k0_t[b] + 1) * split) - l0 == split);
  const int before = (first_partial && s > 0) ? 1 : 0;  // partial splits ahead of s
  int pos;
  if (t1 - t0 == split) {
    pos = fbase[b] + kvh * nf + (s - before);
  } else {
    // partial items follow the full ones, larger chunk counts first (the
    // order inside one count is immaterial)
    const int nch = (t1 - (t0 & ~15) + 15) >> 4;
    int32_t* boff = tab + attn_bucket_offset(batch);
    pos = fbase[batch] + boff[nch] + atomicAdd(boff + RSTR_NCH + nch, 1);
  }
  items[pos] = int4{b | (kvh << 20), t0, t1, i};
}

// k_attn_prep and k_attn_items in one workgroup, for batches of up to 1024
// lanes: the lane tables are written to `tab` as k_attn_prep writes them (the
// split and merge kernels read them), and the work list is built from LDS
// copies of the lane prefix, with the partial items' buckets and fill cursors
// in LDS.  One workgroup per geometry, so the windowed and the global layers'
// tables of a step take one launch.  The per-lane and per-item rules are
// those of the two kernels; the list is the same up to the order inside one
// partial bucket, which no consumer depends on.
struct AttnListArgs {
  int window[2], R[2];
  int32_t* tab[2];
  int4* items[2];
};
__global__ __launch_bounds__(1024) void k_attn_list(int batch, int split, int n_kv, int max_items,
                                                    const int32_t* __restrict__ lengths, AttnListArgs args) {
  __shared__ int32_t s_a[1024], s_f[1024], s_p[1024], s_h[RSTR_NCH], s_cur[RSTR_NCH];
  __shared__ int32_t s_lo[1024], s_k0[1024], s_ns[1024], s_len[1024], s_base[1025], s_fb[1025];
  const int gsel = blockIdx.x;
  const int window = args.window[gsel], R = args.R[gsel];
  int32_t* tab = args.tab[gsel];
  int4* items = args.items[gsel];
  const int tid = threadIdx.x;
  for (int i = tid; i < RSTR_NCH; i += 1024) {
    s_h[i] = 0;
    s_cur[i] = 0;
  }
  __syncthreads();
  // ---- lane tables (k_attn_prep, one chunk of lanes)
  const int b = tid;
  int l0 = 0, kk0 = 0, n = 0, f = 0, len = 0;
  if (b < batch) {
    len = lengths[b];
    if (len > 0) {
      l0 = window > 0 ? max(0, len - window) : 0;
      kk0 = l0 / split;
      n = (len - 1) / split - kk0 + 1;
      const int f_t1 = min(len, (kk0 + 1) * split);
      const bool first_full = l0 == kk0 * split && f_t1 - l0 == split;
      const bool last_full = len % split == 0;
      f = n == 1 ? (first_full ? 1 : 0) : n - (first_full ? 0 : 1) - (last_full ? 0 : 1);
      if (!first_full) atomicAdd(&s_h[(f_t1 - (l0 & ~15) + 15) >> 4], n_kv);
      if (n > 1 && !last_full) {
        const int lt0 = (kk0 + n - 1) * split;
        atomicAdd(&s_h[(len - (lt0 & ~15) + 15) >> 4], n_kv);
      }
    }
  }
  const int32_t va = b < batch ? n * n_kv : 0;
  const int32_t vf = b < batch ? f * n_kv : 0;
  const int32_t vp = va - vf;
  s_a[tid] = va;
  s_f[tid] = vf;
  s_p[tid] = vp;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int32_t ta = tid >= off ? s_a[tid - off] : 0;
    const int32_t tf = tid >= off ? s_f[tid - off] : 0;
    const int32_t tp = tid >= off ? s_p[tid - off] : 0;
    __syncthreads();
    s_a[tid] += ta;
    s_f[tid] += tf;
    s_p[tid] += tp;
    __syncthreads();
  }
  int32_t tot_a = s_a[1023], tot_f = s_f[1023], tot_p = s_p[1023];
  int32_t base_b = s_a[tid] - va, fb_b = s_f[tid] - vf, pb_b = s_p[tid] - vp;
  // more items than the list holds (descriptors the host validation rejects):
  // no attention work, every output 0 (as k_attn_prep)
  const bool over = tot_a > max_items;
  if (over) {
    n = 0;
    base_b = fb_b = pb_b = 0;
    tot_a = tot_f = tot_p = 0;
  }
  if (b < batch) {
    tab[b] = l0;
    tab[batch + b] = kk0;
    tab[2 * batch + b] = n;
    tab[3 * batch + b] = base_b;
    tab[4 * batch + 1 + b] = fb_b;
    tab[5 * batch + 2 + b] = pb_b;
  }
  s_lo[tid] = l0;
  s_k0[tid] = kk0;
  s_ns[tid] = n;
  s_len[tid] = len;
  s_base[tid] = base_b;
  s_fb[tid] = fb_b;
  __syncthreads();  // the scans' arrays are read before they are reused below
  if (over)
    for (int i = tid; i < RSTR_NCH; i += 1024) s_h[i] = 0;
  if (tid == 0) {
    s_base[batch] = tot_a;
    s_fb[batch] = tot_f;
    tab[3 * batch + batch] = tot_a;
    tab[4 * batch + 1 + batch] = tot_f;
    tab[5 * batch + 2 + batch] = tot_p;
    const int arm = attn_static_rounds(tot_a, R) * R;
    tab[attn_ctl_offset(batch)] = arm;
    tab[attn_ctl_offset(batch) + 1] = arm;
  }
  __syncthreads();
  // partial items by decreasing chunk count: boff[c] = the partial items of
  // all counts above c (exclusive suffix sum; thread r holds count NCH-1-r)
  static_assert(RSTR_NCH <= 1024, "one count per thread");
  const int32_t hv = tid < RSTR_NCH ? s_h[RSTR_NCH - 1 - tid] : 0;
  s_a[tid] = hv;
  __syncthreads();
  for (int off = 1; off < RSTR_NCH; off <<= 1) {
    const int32_t t = tid >= off ? s_a[tid - off] : 0;
    __syncthreads();
    s_a[tid] += t;
    __syncthreads();
  }
  int32_t* s_boff = s_p;  // the last scan's array is free again
  if (tid < RSTR_NCH) s_boff[RSTR_NCH - 1 - tid] = s_a[tid] - hv;
  __syncthreads();
  // ---- the work list (k_attn_items)
  for (int i = tid; i < tot_a; i += 1024) {
    int bl = 0, hi = batch;
    while (hi - bl > 1) {
      const int mid = (bl + hi) >> 1;
      if (s_base[mid] <= i) bl = mid; else hi = mid;
    }
    const int ns = s_ns[bl];
    const int rel = i - s_base[bl];
    const int kvh = rel / ns;
    const int sp = rel % ns;
    const int ln = s_len[bl];
    const int k = s_k0[bl] + sp;
    const int t0 = max(s_lo[bl], k * split), t1 = min(ln, (k + 1) * split);
    const int nf = (s_fb[bl + 1] - s_fb[bl]) / n_kv;
    const int lb = s_lo[bl];
    const bool first_partial = !(lb == s_k0[bl] * split && min(ln, (s_k0[bl] + 1) * split) - lb == split);
    const int before = (first_partial && sp > 0) ? 1 : 0;
    int pos;
    if (t1 - t0 == split) {
      pos = s_fb[bl] + kvh * nf + (sp - before);
    } else {
      const int nch = (t1 - (t0 & ~15) + 15) >> 4;
      pos = tot_f + s_boff[nch] + atomicAdd(&s_cur[nch], 1);
    }
    items[pos] = int4{bl | (kvh << 20), t0, t1, i};
  }
}

// The step's work lists of up to two geometries (windowed and global layers)
// sharing lengths, split and max_items: one launch for batches of up to 1024
// lanes, else k_attn_prep + k_attn_items per geometry.
hipError_t launch_attn_lists(hipStream_t st, const AttnGeom* g, int n_geo, const int32_t* lengths,
                             int32_t* lane_tab, size_t tab_stride, int max_items) {
  if (n_geo < 1 || n_geo > 2) return hipErrorInvalidValue;
  if (g[0].batch > 1024) {
    for (int w = 0; w < n_geo; w++) {
      const hipError_t e = launch_attn_prep(st, g[w], lengths, lane_tab + w * tab_stride, max_items);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  AttnListArgs a{};
  for (int w = 0; w < n_geo; w++) {
    if (g[w].batch != g[0].batch || g[w].split != g[0].split || g[w].n_kv != g[0].n_kv) return hipErrorInvalidValue;
    const int R = attn_grid(g[w], max_items);
    if (R <= 0) return hipErrorInvalidValue;
    if (g[w].n_kv >= (1 << 11)) return hipErrorInvalidValue;
    a.window[w] = g[w].window;
    a.R[w] = R;
    a.tab[w] = lane_tab + w * tab_stride;
    a.items[w] = reinterpret_cast<int4*>(a.tab[w] + attn_items_offset(g[w].batch));
  }
  hipLaunchKernelGGL(k_attn_list, dim3(n_geo), dim3(1024), 0, st, g[0].batch, g[0].split, g[0].n_kv, max_items,
                     lengths, a);
  return hipGetLastError();
}

hipError_t launch_attn_prep(hipStream_t st, const AttnGeom& g, const int32_t* lengths,
                            int32_t* lane_tab, int max_items) {
  const int R = attn_grid(g, max_items);
  if (R <= 0) return hipErrorInvalidValue;
  if (g.batch >= (1 << 20) || g.n_kv >= (1 << 11)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_attn_prep, dim3(1), dim3(1024), 0, st, g.batch, g.split, g.window, g.n_kv, R,
                     max_items, lengths, lane_tab);
  hipLaunchKernelGGL(k_attn_items, dim3((max_items + 255) / 256), dim3(256), 0, st, g.batch, g.n_kv, g.split,
                     lengths, lane_tab, reinterpret_cast<int4*>(lane_tab + attn_items_offset(g.batch)));
  return hipGetLastError();
}

// Canonical split partial.  QK: LPT lanes per token, lane j owns 8-dim chunks
// c = j + LPT*i whose slices are c mod 16; slices merge by the fixed tree
// (bit 3, 2, 1, 0 of the slice index), the last levels across lanes.
// Softmax: m = max, p = exp(s - m).  PV: lane group g (16 lanes) takes tokens
// t = g mod 4 in order, each lane owns a fixed set of dims; groups merge
// ((0+1)+(2+3)).
//
// Memory path: one wave per work item streams the item's K rows and then its
// V rows in chunks of 16 tokens through a ring of RB LDS buffers, filled by
// direct-to-LDS loads (global_load_lds_dwordx4) issued RB-1 chunks ahead, so
// a wave keeps up to (RB-1) * 16 rows in flight without holding them in
// registers.  A 16-byte piece p of token row r lands at LDS slot
// r*NP + (p ^ swz(r)); the swizzle makes both the QK reads (LPT lanes per
// row) and the PV reads (16 lanes per row) hit 16 distinct bank groups.
template <int HD, int LPT>
__device__ __forceinline__ int attn_swz(int r) {
  constexpr int NP = HD / 8;
  if constexpr (NP >= 16) return (r % (16 / LPT)) * LPT;
  else return ((r >> 1) & 1) * 4;  // HD = 64, LPT = 4
}

// Cache policy of the page stream's loads: non-temporal (the gfx950 `nt`
// bit).  Every K/V row of a layer is read once per step, so its lines are
// marked to leave L2 first instead of displacing the data the step reuses
// (work list, page tables, split partials).  On MI355X this lifts the split
// kernel from 5.1 to 5.5 TB/s at 128 lanes (a plain read of the same pages:
// 6.1 -> 6.9 TB/s).
#define RSTR_KV_POLICY 2
// Split partial stores: written through to memory (the gfx950 `sc1` bit).
#define RSTR_PART_POLICY 16
// Word 3 of a raw buffer resource on gfx950 (32-bit data format).
#define RSTR_BUF_DW3 0x00020000

// Geometry of one work item (all values wave-uniform).
struct AttnItem {
  int b, kvh, idx, t0, t1, T0, nch;
};

// Item fields are wave-uniform; readfirstlane keeps them in scalar registers
// so the table lookups stay scalar loads (a vector load here would make the
// compiler wait for every outstanding DMA).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Round k of this wave's share of the step's work list (positions k*R + w,
// then k*R + R-1-w, alternating).  The position is wave-uniform, so this is
// one scalar load.  Prefetched entries stay raw until used, so no wait is
// placed at the load.
// Rounds below ks are static; later ones claim the next unclaimed list
// position from the launch's counter (armed to ks*R), so waves that run ahead
// take over the tail.  Entry x < 0: the wave's sequence has ended.  Claims
// are device-scope atomics on one word, which serialise: when every wave
// claims at once (a list of one or two rounds, or a claim for the second
// round made as each wave starts) they cost more than the imbalance they
// remove, so such lists are static throughout (attn_static_rounds).
__device__ __forceinline__ int4 attn_item_fetch(const int4* __restrict__ items, int k, int ks, int n,
                                                int* __restrict__ ctr) {
  const int R = gridDim.x, w = blockIdx.x;
  if (k < ks) {
    const int pos = k * R + ((k & 1) ? R - 1 - w : w);
    return pos < n ? items[pos] : int4{-1, 0, 0, 0};
  }
  if (ks * R >= n) return int4{-1, 0, 0, 0};  // no list position is left to claim
  int v = 0;
  if (threadIdx.x == 0) v = atomicAdd(ctr, 1);
  const int pos = uni(v);
  if (pos < n) return items[pos];
  return int4{-1, 0, 0, 0};
}
__device__ __forceinline__ AttnItem attn_item_make(int4 d) {
  AttnItem it;
  it.b = uni(d.x & 0xFFFFF);
  it.kvh = uni(d.x >> 20);
  it.idx = uni(d.w);
  it.t0 = uni(d.y);
  it.t1 = uni(d.z);
  it.T0 = it.t0 & ~15;
  it.nch = (it.t1 - it.T0 + 15) >> 4;
  return it;
}

template <int HD, int G, int LPT, bool PG16, int RB>
__global__ __launch_bounds__(64) void k_attn_split(
    int n_kv, int page_size, int ps_shift, int pps, float scale,
    const float* __restrict__ q, const uint16_t* __restrict__ kp, const uint16_t* __restrict__ vp,
    const int32_t* __restrict__ page_table, const int32_t* __restrict__ n_items,
    const int4* __restrict__ items, int* __restrict__ ctr, float* __restrict__ part) {
  constexpr int NP = HD / 8;             // 16-byte pieces per row
  constexpr int CT = 16;                 // tokens per chunk
  constexpr int CU16 = CT * NP;          // 16-byte units per chunk
  constexpr int LPC = CU16 / 64;         // DMA instructions per chunk
  constexpr int NCL = NP / LPT;          // QK pieces per lane
  constexpr int NSL = 16 / LPT;          // slice slots per lane
  constexpr int TPP = 64 / LPT;          // tokens per QK pass
  constexpr int PPL = NP >= 16 ? NP / 16 : 1;   // PV pieces per lane (HD 64: half a piece)
  constexpr int DPL = HD / 16;           // PV dims per lane
  constexpr int WAIT_STEADY = ((LPC * (RB - 1)) & 0xF) | (((LPC * (RB - 1)) >> 4) << 14) | 0x0F70;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  constexpr int QB = (G * HD * 4 + 1023) / 1024;  // 1 KB DMA blocks of one kv group's query
  u32x4* ring = reinterpret_cast<u32x4*>(smem);                        // [RB][CU16]
  u32x4* qlds = ring + RB * CU16;                                       // [QB][64]
  float* sc = reinterpret_cast<float*>(qlds + QB * 64);                 // [split][G]
  const int lane = threadIdx.x;
  const int kvr = n_kv * HD;
  const int ts = lane / LPT, j = lane % LPT;
  // Lane j of a token's LPT lanes owns 8-dim chunks jp + LPT*i.  For LPT = 8
  // the order 0 1 2 3 7 6 5 4 puts slices s and s^4 in mirrored lanes of the
  // 8-lane group, so the bit-2 merge is one DPP half-row mirror (bits 1 and 0
  // stay quad permutes); for other LPT, jp = j.
  const int jp = (LPT == 8 && j >= 4) ? 11 - j : j;
  static_assert(CT % TPP == 0, "a QK pass covers a whole number of chunk rows");
  constexpr int NPASS = CT / TPP;            // QK passes per chunk
  constexpr int QPB = NPASS >= 2 ? 2 : 1;    // passes per batch
  const int grp = lane >> 4, e16 = lane & 15;
  // per-lane DMA geometry: row within the chunk and element offset of the
  // lane's 16-byte piece for each of the chunk's LPC load instructions
  int dma_r[LPC], dma_off[LPC];
  uint32_t dma_boff[LPC];  // byte offset from the chunk's first row (one page)
#pragma unroll
  for (int u = 0; u < LPC; u++) {
    const int pos = u * 64 + lane;
    dma_r[u] = pos / NP;
    dma_off[u] = ((pos % NP) ^ attn_swz<HD, LPT>(dma_r[u])) * 8;
    dma_boff[u] = (uint32_t)(dma_r[u] * kvr + dma_off[u]) * 2u;
  }

  // This wave's work: ks static rounds of the list, then claims.  Round 0 is
  // always static: the wave's first entry (list position w) is loaded
  // together with the item count instead of after it.
  const int4 first_raw = items[blockIdx.x];
  const int n_tot = uni(*n_items);
  const int ks = attn_static_rounds(n_tot, (int)gridDim.x);
  int pk = 1;  // rounds fetched
  if ((int)blockIdx.x >= n_tot) return;
  const int4 first = first_raw;
  // Issue priority by progress: a SIMD's two waves otherwise share issue by
  // age, so the older one runs ahead through the static rounds and the younger
  // one sets the launch's end.  Each wave starts at priority 3 and steps down
  // with every item it completes, so a wave that has fallen behind wins issue
  // until it catches up (config5: 234 -> 228.5 us per split + merge).
  __builtin_amdgcn_s_setprio(3);
  int items_done = 0;

  // One continuous stream per wave: the positions of an item are its K
  // chunks, then its V chunks; the producer runs RB-1 positions ahead of the
  // consumer across item boundaries, so the ring never drains between items.
  // Entries the producer fetched and the consumer has not started wait in a
  // three-deep FIFO (the producer is at most two items and one prefetch ahead).
  int ppos = 0;                         // producer position within gp
  bool pdone = false;                   // producer has issued everything
  AttnItem gp = attn_item_make(first);  // producer's item
  int4 gpn = attn_item_fetch(items, pk++, ks, n_tot, ctr);  // the item after gp
  AttnItem gc = gp;                     // consumer's item
  int4 fq0 = gpn, fq1 = gpn, fq2 = gpn;
  int fqn = gpn.x >= 0 ? 1 : 0;
  int pslot = 0;  // ring slot of the producer's next chunk
  // PG16: page_size is a power of two and a multiple of 16, so a chunk lies in
  // one page; pg_next is the page of the producer's next chunk.
  const uint32_t row_bytes = (uint32_t)kvr * 2u;
  const uint32_t page_bytes = (uint32_t)page_size * row_bytes;
  int pg_next = 0;
  if constexpr (PG16) pg_next = page_table[(size_t)gp.b * pps + (gp.T0 >> ps_shift)];

#define RSTR_ATTN_ISSUE()                                                                         \
  do {                                                                                            \
    const bool isk_ = ppos < gp.nch;                                                              \
    const int c_ = isk_ ? ppos : ppos - gp.nch;                                                   \
    const uint16_t* src_ = (isk_ ? kp : vp) + gp.kvh * HD;                                        \
    u32x4* dst_ = ring + pslot * CU16;                                                            \
    const int tb_ = gp.T0 + c_ * CT;                                                              \
    if constexpr (PG16) {                                                                         \
      const char* cb_ = reinterpret_cast<const char*>(src_) + (uint64_t)(uint32_t)pg_next * page_bytes + \
                        (uint32_t)(tb_ & (page_size - 1)) * row_bytes;                            \
      _Pragma("unroll") for (int u = 0; u < LPC; u++)                                             \
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(cb_ + dma_boff[u]),        \
                                         RSTR_LDS_PTR(dst_ + u * 64), 16, 0, RSTR_KV_POLICY);     \
    } else {                                                                                      \
      const int32_t* prow_ = page_table + (size_t)gp.b * pps;                                     \
      _Pragma("unroll") for (int u = 0; u < LPC; u++) {                                           \
        const int t_ = min(max(tb_ + dma_r[u], gp.t0), gp.t1 - 1);                                \
        const int page_ = prow_[t_ / page_size];                                                  \
        const uint16_t* g_ = src_ + ((size_t)page_ * page_size + (t_ % page_size)) * kvr + dma_off[u]; \
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(g_), RSTR_LDS_PTR(dst_ + u * 64), 16, 0, \
                                         RSTR_KV_POLICY);                                         \
      }                                                                                           \
    }                                                                                             \
    pslot = pslot == RB - 1 ? 0 : pslot + 1;                                                      \
    if (++ppos == 2 * gp.nch) {                                                                   \
      ppos = 0;                                                                                   \
      if (gpn.x >= 0) {                                                                           \
        gp = attn_item_make(gpn);                                                                 \
        gpn = attn_item_fetch(items, pk++, ks, n_tot, ctr);                                       \
        if (gpn.x >= 0) {                                                                         \
          if (fqn == 0) fq0 = gpn;                                                                \
          else if (fqn == 1) fq1 = gpn;                                                           \
          else fq2 = gpn;                                                                         \
          fqn++;                                                                                  \
        }                                                                                         \
      } else {                                                                                    \
        pdone = true;                                                                             \
      }                                                                                           \
    }                                                                                             \
    if constexpr (PG16) {                                                                         \
      if (!pdone) {                                                                               \
        const int cn_ = ppos < gp.nch ? ppos : ppos - gp.nch;                                     \
        pg_next = page_table[(size_t)gp.b * pps + ((gp.T0 + cn_ * CT) >> ps_shift)];              \
      }                                                                                           \
    }                                                                                             \
  } while (0)

  for (int k = 0; k < RB - 1; k++)
    if (!pdone) RSTR_ATTN_ISSUE();

  // consumer
  int cpos = 0, consumed = 0, cslot = 0;
  float qv[G][NCL][8];
  // A kv group's G query rows are contiguous: they reach LDS by QB DMA
  // instructions (lanes past the end re-read the last piece).
#define RSTR_ATTN_DMA_Q(IT)                                                                       \
  do {                                                                                            \
    const float* qg_ = q + ((size_t)(IT).b * (n_kv * G) + (IT).kvh * G) * HD;                     \
    _Pragma("unroll") for (int u = 0; u < QB; u++) {                                              \
      const int pc_ = min(u * 64 + lane, G * HD / 4 - 1);                                         \
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(qg_ + 4 * pc_),              \
                                       RSTR_LDS_PTR(qlds + u * 64), 16, 0, 0);                    \
    }                                                                                             \
  } while (0)
#define RSTR_ATTN_READ_Q()                                                                        \
  do {                                                                                            \
    const float* qf_ = reinterpret_cast<const float*>(qlds);                                      \
    _Pragma("unroll") for (int h = 0; h < G; h++)                                                 \
      _Pragma("unroll") for (int i = 0; i < NCL; i++) {                                           \
        const int cch = jp + LPT * i;                                                             \
        const f4 a = *reinterpret_cast<const f4*>(qf_ + h * HD + 8 * cch);                        \
        const f4 bq = *reinterpret_cast<const f4*>(qf_ + h * HD + 8 * cch + 4);                   \
        _Pragma("unroll") for (int e = 0; e < 4; e++) { qv[h][i][e] = a[e]; qv[h][i][4 + e] = bq[e]; } \
      }                                                                                           \
  } while (0)
  RSTR_ATTN_DMA_Q(gc);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): first query and first chunks
  __asm__ __volatile__("" ::: "memory");
  RSTR_ATTN_READ_Q();
  int q_dma_step = -RB;  // consumer step at which the next query DMA was issued
  float mx[G], o[G][DPL], l[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    mx[h] = -__builtin_inff();
    l[h] = 0.0f;
#pragma unroll
    for (int d = 0; d < DPL; d++) o[h][d] = 0.0f;
  }

  while (true) {
    if (!pdone) {
      // the ring slot being refilled was last read one step ago; its LDS
      // reads (and the prefetched page id) have all returned
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      RSTR_ATTN_ISSUE();
      __builtin_amdgcn_s_waitcnt(WAIT_STEADY);  // position `consumed` has landed
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the stream is draining
    }
    __asm__ __volatile__("" ::: "memory");
    const u32x4* buf = ring + cslot * CU16;
    const int t0 = gc.t0, t1 = gc.t1;
    if (cpos < gc.nch) {
      // ---- QK over the 16 rows of this chunk --------------------------------
      // Passes run in batches of QPB: every LDS read of a batch is issued
      // before its fmas, and the cross-lane merges of the batch's G*QPB dots
      // are independent DPP operations.
#pragma unroll
      for (int pb = 0; pb < NPASS; pb += QPB) {
        float sv[QPB][G][NSL];
#pragma unroll
        for (int ps = 0; ps < QPB; ps++)
#pragma unroll
          for (int h = 0; h < G; h++)
#pragma unroll
            for (int u = 0; u < NSL; u++) sv[ps][h][u] = 0.0f;
        h8 kv[QPB][NCL];
#pragma unroll
        for (int ps = 0; ps < QPB; ps++) {
          const int r = (pb + ps) * TPP + ts;
#pragma unroll
          for (int i = 0; i < NCL; i++) {
            const int piece = jp + LPT * i;
            kv[ps][i] = __builtin_bit_cast(h8, buf[r * NP + (piece ^ attn_swz<HD, LPT>(r))]);
          }
        }
#pragma unroll
        for (int ps = 0; ps < QPB; ps++)
#pragma unroll
          for (int i = 0; i < NCL; i++)
#pragma unroll
            for (int h = 0; h < G; h++)
#pragma unroll
              for (int e = 0; e < 8; e++)
                sv[ps][h][i % NSL] = __builtin_fmaf(qv[h][i][e], (float)kv[ps][i][e], sv[ps][h][i % NSL]);
#pragma unroll
        for (int ps = 0; ps < QPB; ps++) {
          const int r = (pb + ps) * TPP + ts;
          const int t = gc.T0 + cpos * CT + r;
          const bool valid = t >= t0 && t < t1;
          float scv[G];
#pragma unroll
          for (int h = 0; h < G; h++) {
            float v;
            if constexpr (LPT == 4) v = (sv[ps][h][0] + sv[ps][h][2]) + (sv[ps][h][1] + sv[ps][h][3]);
            else if constexpr (LPT == 8) v = sv[ps][h][0] + sv[ps][h][1];
            else v = sv[ps][h][0];
            if constexpr (LPT >= 16) v = v + xor_lane<8>(v);
            if constexpr (LPT == 8) v = v + half_mirror_lane(v);  // slices jp and jp ^ 4
            else if constexpr (LPT >= 16) v = v + xor_lane<4>(v);
            v = v + xor_lane<2>(v);
            v = v + xor_lane<1>(v);
            scv[h] = v * scale;
            if (valid) mx[h] = fmaxf(mx[h], scv[h]);
          }
          if (valid && j == 0) {
            float* dst = sc + (size_t)(t - t0) * G;
            if constexpr (G % 4 == 0) {
#pragma unroll
              for (int h4 = 0; h4 < G; h4 += 4)
                *reinterpret_cast<f4*>(dst + h4) = f4{scv[h4], scv[h4 + 1], scv[h4 + 2], scv[h4 + 3]};
            } else {
#pragma unroll
              for (int h = 0; h < G; h++) dst[h] = scv[h];
            }
          }
        }
      }
      if (cpos == gc.nch - 1) {
        // ---- softmax numerators over the whole split ----------------------------
#pragma unroll
        for (int h = 0; h < G; h++) mx[h] = wave_max(mx[h]);
        // The workgroup is this one wave, whose LDS accesses execute in
        // program order: a compiler barrier orders the score writes and reads
        // (a workgroup barrier would also wait for every DMA in flight).
        __asm__ __volatile__("" ::: "memory");
        const int nt = t1 - t0;
        for (int i = lane; i < nt; i += 64)
#pragma unroll
          for (int h = 0; h < G; h++) sc[i * G + h] = dexp(sc[i * G + h] - mx[h]);
        __asm__ __volatile__("" ::: "memory");
        // the next item's query: its DMA lands while this item's V chunks run
        // (qv itself is reloaded from LDS when the next item starts)
        if (fqn > 0) {
          const AttnItem gn = attn_item_make(fq0);
          RSTR_ATTN_DMA_Q(gn);
          q_dma_step = consumed;
        }
      }
    } else {
      // ---- PV over the 16 rows of this chunk: 4 rounds of one row per group ----
      // Interior chunks hold only visible rows.  In the first and last chunk
      // a row outside [t0, t1) contributes p = 0 times v = 0, which leaves
      // o and l unchanged (they are never -0), without branching per lane.
      const int c = cpos - gc.nch;
      const bool edge = (c == 0) || (c == gc.nch - 1);
#define RSTR_PV_ROUNDS(MASK)                                                                      \
      _Pragma("unroll") for (int rd = 0; rd < CT / 4; rd++) {                                     \
        const int r = rd * 4 + grp;                                                               \
        const int t = gc.T0 + c * CT + r;                                                         \
        const bool ok = !(MASK) || (t >= t0 && t < t1);                                           \
        float vv[DPL];                                                                            \
        if constexpr (NP >= 16) {                                                                 \
          _Pragma("unroll") for (int pp = 0; pp < PPL; pp++) {                                    \
            const int piece = e16 + 16 * pp;                                                      \
            const h8 hv = __builtin_bit_cast(h8, buf[r * NP + (piece ^ attn_swz<HD, LPT>(r))]);   \
            _Pragma("unroll") for (int e = 0; e < 8; e++) vv[pp * 8 + e] = ok ? (float)hv[e] : 0.0f; \
          }                                                                                       \
        } else {                                                                                  \
          const int piece = e16 >> 1;                                                             \
          const u32x4 pv = buf[r * NP + (piece ^ attn_swz<HD, LPT>(r))];                          \
          const u32x2 half = (e16 & 1) ? u32x2{pv[2], pv[3]} : u32x2{pv[0], pv[1]};               \
          const h4 hv = __builtin_bit_cast(h4, half);                                             \
          _Pragma("unroll") for (int e = 0; e < 4; e++) vv[e] = ok ? (float)hv[e] : 0.0f;         \
        }                                                                                         \
        float pr[G];                                                                              \
        const float* ps_ = sc + (size_t)(ok ? t - t0 : 0) * G;                                    \
        if constexpr (G % 4 == 0) {                                                               \
          _Pragma("unroll") for (int h4 = 0; h4 < G; h4 += 4) {                                   \
            const f4 p4 = *reinterpret_cast<const f4*>(ps_ + h4);                                 \
            _Pragma("unroll") for (int e = 0; e < 4; e++) pr[h4 + e] = ok ? p4[e] : 0.0f;         \
          }                                                                                       \
        } else {                                                                                  \
          _Pragma("unroll") for (int h = 0; h < G; h++) pr[h] = ok ? ps_[h] : 0.0f;               \
        }                                                                                         \
        _Pragma("unroll") for (int h = 0; h < G; h++) {                                           \
          l[h] = l[h] + pr[h];                                                                    \
          _Pragma("unroll") for (int d = 0; d < DPL; d++) o[h][d] = __builtin_fmaf(pr[h], vv[d], o[h][d]); \
        }                                                                                         \
      }
      if (edge) {
        RSTR_PV_ROUNDS(true)
      } else {
        RSTR_PV_ROUNDS(false)
      }
#undef RSTR_PV_ROUNDS
    }
    consumed++;
    cslot = cslot == RB - 1 ? 0 : cslot + 1;
    if (++cpos < 2 * gc.nch) continue;
    // ---- item complete: combine lane groups, write the partial ---------------
#pragma unroll
    for (int h = 0; h < G; h++) {
      l[h] = xor_add<32>(xor_add<16>(l[h]));
#pragma unroll
      for (int d = 0; d < DPL; d++) {
        o[h][d] = xor_add<32>(xor_add<16>(o[h][d]));
      }
    }
    // Every lane group now holds the whole partial; group grp writes the
    // records of heads grp, grp + 4, ... with 16-byte stores from all its
    // lanes.  The stores are written through (sc1): the partials are read
    // only by the merge launch, and lines held back in L2 and written back
    // while the page stream runs cost read bandwidth.
    {
      constexpr int PF = attn_part_floats(HD);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(part + (size_t)gc.idx * G * PF, 0, G * PF * 4, RSTR_BUF_DW3);
#pragma unroll
      for (int h0 = 0; h0 < G; h0 += 4) {
        const int h = h0 + grp;
        if (h < G) {
          float ov[DPL], mh = mx[h0], lh = l[h0];
#pragma unroll
          for (int d = 0; d < DPL; d++) ov[d] = o[h0][d];
#pragma unroll
          for (int k = 1; k < 4 && h0 + k < G; k++) {
            if (grp == k) {
#pragma unroll
              for (int d = 0; d < DPL; d++) ov[d] = o[h0 + k][d];
              mh = mx[h0 + k];
              lh = l[h0 + k];
            }
          }
          const int rb = h * PF * 4;  // record byte offset
          if constexpr (NP >= 16) {
#pragma unroll
            for (int pp = 0; pp < PPL; pp++)
#pragma unroll
              for (int q4 = 0; q4 < 2; q4++)
                __builtin_amdgcn_raw_buffer_store_b128(
                    u32x4{__builtin_bit_cast(uint32_t, ov[pp * 8 + q4 * 4]), __builtin_bit_cast(uint32_t, ov[pp * 8 + q4 * 4 + 1]),
                          __builtin_bit_cast(uint32_t, ov[pp * 8 + q4 * 4 + 2]), __builtin_bit_cast(uint32_t, ov[pp * 8 + q4 * 4 + 3])},
                    rs, rb + ((e16 + 16 * pp) * 8 + q4 * 4) * 4, 0, RSTR_PART_POLICY);
          } else {
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__builtin_bit_cast(uint32_t, ov[0]), __builtin_bit_cast(uint32_t, ov[1]),
                      __builtin_bit_cast(uint32_t, ov[2]), __builtin_bit_cast(uint32_t, ov[3])},
                rs, rb + e16 * 16, 0, RSTR_PART_POLICY);
          }
          if (e16 == 0)
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{__builtin_bit_cast(uint32_t, mh), __builtin_bit_cast(uint32_t, lh)},
                                                  rs, rb + HD * 4, 0, RSTR_PART_POLICY);
        }
      }
    }
    if (++items_done == 1) __builtin_amdgcn_s_setprio(2);
    else if (items_done == 2) __builtin_amdgcn_s_setprio(1);
    else if (items_done == 3) __builtin_amdgcn_s_setprio(0);
    if (fqn == 0) break;
    cpos = 0;
    gc = attn_item_make(fq0);
    fq0 = fq1;
    fq1 = fq2;
    fqn--;
    // the query DMA is complete once a position issued after it has been
    // waited for; position p is issued at consumer step p - (RB - 1)
    if (consumed - 1 < q_dma_step + RB) __builtin_amdgcn_s_waitcnt(0x0F70);
    __asm__ __volatile__("" ::: "memory");
    RSTR_ATTN_READ_Q();
#pragma unroll
    for (int h = 0; h < G; h++) {
      mx[h] = -__builtin_inff();
      l[h] = 0.0f;
#pragma unroll
      for (int d = 0; d < DPL; d++) o[h][d] = 0.0f;
    }
  }
#undef RSTR_ATTN_ISSUE
#undef RSTR_ATTN_DMA_Q
#undef RSTR_ATTN_READ_Q
}

// ---- qkv post-processing inside the few-item kernel (AttnQkv) --------------------
// One head of row `src`'s qkv output with k_qkv_post's arithmetic: lane l <
// HD/4 holds elements 4l..4l+3 (slices added in the canonical tree), then the
// optional RMS norm over the head.
template <int HD>
__device__ __forceinline__ f4 qkv_head(const AttnQkv& qk, size_t src, const float* gn, int lane) {
  constexpr int HD4 = HD / 4;
  const bool have = lane < HD4;
  const int cc = have ? lane : 0;
  f4 v;
  if (qk.y.n == 1) v = sl_get<1>(qk.y, src + 4 * cc);
  else if (qk.y.n == 2) v = sl_get<2>(qk.y, src + 4 * cc);
  else v = sl_get<4>(qk.y, src + 4 * cc);
  if (gn) {
    const f4 gg = *reinterpret_cast<const f4*>(gn + 4 * cc);
    float a = 0.0f;
    if (have) {
      a = __builtin_fmaf(v[0], v[0], a);
      a = __builtin_fmaf(v[1], v[1], a);
      a = __builtin_fmaf(v[2], v[2], a);
      a = __builtin_fmaf(v[3], v[3], a);
    }
    // HD/4 <= 64 chunks: lane l holds slot l alone, and the tree over 64
    // lanes equals the 256-slot tree (the other slots are +0)
    const float r = rms_scale(wave_tree_sum(a), HD, qk.eps);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = (v[i] * r) * (qk.goff + gg[i]);
  }
  return v;
}

// The item's q heads (wave w: heads w, w+4, ...) into qst[G][HD], rotated at the
// row's position; the item holding the lane's newest token also writes that
// token's K (wave 0: norm, RoPE) and V (wave 1) to the pages at the slot.
// Every write is complete and visible to the workgroup on return.
template <int HD, int G>
__device__ void attn_qkv_prologue(const AttnQkv& qk, const AttnItem& it, int n_kv, int lane, int wave,
                                  float* qst) {
  constexpr int HD4 = HD / 4, HALF = HD / 2;
  const int kvr = n_kv * HD, qd = n_kv * G * HD;
  const size_t yr = (size_t)it.b * (qd + 2 * kvr);
  const bool have = lane < HD4;
  const int slot = uni(qk.slots[it.b]);
  const bool newest = slot >= 0 && it.t1 == uni(qk.lengths[it.b]);
  const int pos = uni(qk.positions[it.b]);
  float* kst = qst + G * HD;
  for (int h = wave; h < G; h += 4) {
    const f4 v = qkv_head<HD>(qk, yr + (size_t)(it.kvh * G + h) * HD, qk.qn, lane);
    if (have) *reinterpret_cast<f4*>(qst + h * HD + 4 * lane) = v;
  }
  if (newest && wave == 0) {
    const f4 v = qkv_head<HD>(qk, yr + qd + (size_t)it.kvh * HD, qk.kn, lane);
    if (have) *reinterpret_cast<f4*>(kst + 4 * lane) = v;
  }
  if (newest && wave == 1) {
    const f4 v = qkv_head<HD>(qk, yr + qd + kvr + (size_t)it.kvh * HD, nullptr, lane);
    if (have) {
      uint16_t* dst = qk.vpages + (size_t)slot * kvr + it.kvh * HD;
#pragma unroll
      for (int i = 0; i < 4; i++) dst[4 * lane + i] = f2h_bits(v[i]);
    }
  }
  __syncthreads();
  // HF rotate-half: y_i = x_i c - x_{i+h} s, y_{i+h} = x_{i+h} c + x_i s
  const float* ct = qk.cos_t + (size_t)pos * HALF;
  const float* stt = qk.sin_t + (size_t)pos * HALF;
  for (int h = wave; h < G; h += 4)
    for (int i = lane; i < HALF; i += 64) {
      const float a = qst[h * HD + i], b = qst[h * HD + i + HALF], c = ct[i], sn = stt[i];
      qst[h * HD + i] = (a * c) - (b * sn);
      qst[h * HD + i + HALF] = (b * c) + (a * sn);
    }
  if (newest && wave == 0) {
    uint16_t* dst = qk.kpages + (size_t)slot * kvr + it.kvh * HD;
    for (int i = lane; i < HALF; i += 64) {
      const float a = kst[i], b = kst[i + HALF], c = ct[i], sn = stt[i];
      dst[i] = f2h_bits((a * c) - (b * sn));
      dst[i + HALF] = f2h_bits((b * c) + (a * sn));
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the K/V stores are complete
  __syncthreads();                     // rotated q in LDS; the appended row is visible to the DMAs that follow
}

// ---- few-item attention: one workgroup of four waves per item -------------------
// The same canonical order as k_attn_split, for launches whose whole work list
// fits in two rounds of resident workgroups (few lanes, short contexts).  There
// an item's own instruction stream bounds the launch: a single wave spends
// ~0.85 us of dependent QK/PV work per 16-token chunk.  Here four waves share
// each item:
//  - QK: 16 lanes per token (lane j holds pieces j + 16i, i.e. slice j, in
//    order), so each wave scores 4 tokens of a chunk; the slice tree runs on
//    bits 3, 2, 1, 0 as in the one-wave kernel;
//  - the split's max is exchanged through LDS, and all 256 threads run the
//    exp pass;
//  - PV: wave g carries lane group g's chains (tokens t = g mod 4 in order)
//    with 64 lanes of HD/64 dims each; the groups combine as ((0+1)+(2+3))
//    through LDS, the same sums as the one-wave kernel's lane exchanges.
// A ring of RB chunks, each filled by all 256 threads' DMAs, streams the
// item's K then V chunks and drains between items.  Every list position is
// static (attn_static_rounds gives one or two rounds here), so no claims.
//
// QKV: the item's query comes from the qkv projection slices through
// attn_qkv_prologue (q is unused), and the lane's newest K/V row is appended
// by the item that holds it, so no separate qkv launch precedes this one.
// (The QKV form keeps three waves per SIMD for G <= 4: a few kernel-constant
// prologue values then live in scratch and are reloaded once per item.)
template <int HD, int G, int RB, bool QKV = false, bool DIRECT = false>
__global__ __launch_bounds__(256, QKV && G <= 4 ? 3 : 1) void k_attn_split_wg(
    int n_kv, int page_size, int ps_shift, int pps, float scale,
    const float* __restrict__ q, const uint16_t* kp, const uint16_t* vp,
    const int32_t* __restrict__ page_table, const int32_t* __restrict__ n_items,
    const int4* __restrict__ items, float* __restrict__ part, AttnQkv qk, AttnOut ao) {
  constexpr int NP = HD / 8;       // 16-byte pieces per row
  constexpr int CT = 16;           // tokens per chunk
  constexpr int CU16 = CT * NP;    // 16-byte units per chunk
  constexpr int UPT = CU16 / 256;  // DMA units per thread per chunk
  constexpr int NCL = NP / 16;     // QK pieces per lane
  constexpr int DPL = HD / 64;     // PV dims per lane
  constexpr int PF = attn_part_floats(HD);
  static_assert(UPT >= 1 && NCL >= 1 && DPL >= 2, "head dim 128 or 256");
  static_assert(RB * CU16 * 16 >= 4 * G * HD * 4, "the group combine fits in the ring");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  u32x4* ring = reinterpret_cast<u32x4*>(smem);                   // [RB][CU16]
  float* red = reinterpret_cast<float*>(ring + RB * CU16);        // [4][G] wave maxima, then l
  float* qst = red + 4 * G;                                       // [G + 1][HD] q (and K) staging
  float* sc = qst + (G + 1) * HD;                                 // [split][G] scores
  float* comb = reinterpret_cast<float*>(smem);                   // [4][G][HD] o, after PV
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tt = tid >> 4, j = tid & 15;  // QK: token of the chunk, slice
  const int kvr = n_kv * HD;
  const uint32_t row_bytes = (uint32_t)kvr * 2u;
  const uint32_t page_bytes = (uint32_t)page_size * row_bytes;
  const int n_tot = uni(*n_items);
  const int R = gridDim.x, w = blockIdx.x;
  const int ks = attn_static_rounds(n_tot, R);
  for (int k = 0; k < ks; k++) {
    const int pos = k * R + ((k & 1) ? R - 1 - w : w);
    if (pos >= n_tot) continue;
    const AttnItem it = attn_item_make(items[pos]);
    const int npos = 2 * it.nch;
    // The pages of the item's chunks: every wave loads them once per item
    // (lane i holds page pg0 + i + 64 k in pgv[k]) and reads each chunk's
    // page with v_readlane (a lookup per chunk would put a memory latency
    // before every DMA).
    const int pg0 = it.T0 >> ps_shift;
    const int npg = ((it.T0 + (it.nch - 1) * CT) >> ps_shift) - pg0 + 1;
    const int32_t* prow = page_table + (size_t)it.b * pps + pg0;
    constexpr int PGV = (RSTR_NCH + 63) / 64;
    int32_t pgv[PGV];
#pragma unroll
    for (int k = 0; k < PGV; k++) pgv[k] = (k == 0 || 64 * k < npg) && lane + 64 * k < npg ? prow[lane + 64 * k] : 0;
    auto issue = [&](int p) {
      const bool isk = p < it.nch;
      const int c = isk ? p : p - it.nch;
      const int tb = it.T0 + c * CT;
      const int pi = (tb >> ps_shift) - pg0;
      int page = __builtin_amdgcn_readlane(pgv[0], pi & 63);
#pragma unroll
      for (int k = 1; k < PGV; k++)
        if ((pi >> 6) == k) page = __builtin_amdgcn_readlane(pgv[k], pi & 63);
      const char* base = reinterpret_cast<const char*>((isk ? kp : vp) + it.kvh * HD) +
                         (uint64_t)(uint32_t)page * page_bytes + (uint32_t)(tb & (page_size - 1)) * row_bytes;
      u32x4* dst = ring + (p % RB) * CU16;
#pragma unroll
      for (int u = 0; u < UPT; u++) {
        const int un = u * 256 + tid;
        __builtin_amdgcn_global_load_lds(
            reinterpret_cast<const void*>(base + (uint32_t)(un / NP) * row_bytes + (uint32_t)(un % NP) * 16u),
            RSTR_LDS_PTR(dst + u * 256 + wave * 64), 16, 0, RSTR_KV_POLICY);
      }
    };
    // this thread's query pieces: slice j of each head
    float qv[G][NCL][8];
    if constexpr (QKV) {
      attn_qkv_prologue<HD, G>(qk, it, n_kv, lane, wave, qst);
#pragma unroll
      for (int h = 0; h < G; h++)
#pragma unroll
        for (int i = 0; i < NCL; i++) {
          const f4 a = *reinterpret_cast<const f4*>(qst + h * HD + 8 * (j + 16 * i));
          const f4 b4 = *reinterpret_cast<const f4*>(qst + h * HD + 8 * (j + 16 * i) + 4);
#pragma unroll
          for (int e = 0; e < 4; e++) { qv[h][i][e] = a[e]; qv[h][i][4 + e] = b4[e]; }
        }
    } else {
      const float* qg = q + ((size_t)it.b * (n_kv * G) + it.kvh * G) * HD;
#pragma unroll
      for (int h = 0; h < G; h++)
#pragma unroll
        for (int i = 0; i < NCL; i++) {
          const f4 a = *reinterpret_cast<const f4*>(qg + h * HD + 8 * (j + 16 * i));
          const f4 b4 = *reinterpret_cast<const f4*>(qg + h * HD + 8 * (j + 16 * i) + 4);
#pragma unroll
          for (int e = 0; e < 4; e++) { qv[h][i][e] = a[e]; qv[h][i][4 + e] = b4[e]; }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // page ids and the query pieces have arrived
    for (int p = 0; p < RB - 1 && p < npos; p++) issue(p);
    float mx[G], o[G][DPL], l[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
      mx[h] = -__builtin_inff();
      l[h] = 0.0f;
#pragma unroll
      for (int d = 0; d < DPL; d++) o[h][d] = 0.0f;
    }
    for (int p = 0; p < npos; p++) {
      // chunk p has landed for this thread once at most the DMAs of the
      // positions after it (at most RB - 2) are outstanding; its LDS writes
      // (scores, exp values) are done before the barrier
      if (p + RB - 2 < npos) __builtin_amdgcn_s_waitcnt(((UPT * (RB - 2)) & 0xF) | (((UPT * (RB - 2)) >> 4) << 14) | 0x0070);
      else __builtin_amdgcn_s_waitcnt(0x0070);
      __asm__ __volatile__("" ::: "memory");
      __builtin_amdgcn_s_barrier();  // every thread's part of chunk p, and every read of slot (p-1) % RB, is done
      __asm__ __volatile__("" ::: "memory");
      if (p + RB - 1 < npos) issue(p + RB - 1);
      const u32x4* buf = ring + (p % RB) * CU16;
      if (p < it.nch) {
        // ---- QK: token tt of chunk p, slice j -----------------------------------
        const int t = it.T0 + p * CT + tt;
        const bool valid = t >= it.t0 && t < it.t1;
        float sv[G];
#pragma unroll
        for (int h = 0; h < G; h++) sv[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < NCL; i++) {
          const h8 kv = __builtin_bit_cast(h8, buf[tt * NP + j + 16 * i]);
#pragma unroll
          for (int h = 0; h < G; h++)
#pragma unroll
            for (int e = 0; e < 8; e++) sv[h] = __builtin_fmaf(qv[h][i][e], (float)kv[e], sv[h]);
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
          // slice tree inside each 16-lane row, all DPP: row_ror:8 is lane
          // i ^ 8; after that level lanes i and i ^ 8 agree, so row_ror:4
          // delivers the value of lane i ^ 4
          float v = sv[h];
          v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, true));
          v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, true));
          v = v + xor_lane<2>(v);
          v = v + xor_lane<1>(v);
          const float s = v * scale;
          if (valid) mx[h] = fmaxf(mx[h], s);
          if (valid && j == 0) sc[(size_t)(t - it.t0) * G + h] = s;
        }
        if (p == it.nch - 1) {
          // ---- softmax numerators over the split --------------------------------
#pragma unroll
          for (int h = 0; h < G; h++) {
            mx[h] = wave_max(mx[h]);
            if (lane == 0) red[wave * G + h] = mx[h];
          }
          // scores and wave maxima are written (LDS only: the V chunks in
          // flight keep streaming)
          __builtin_amdgcn_s_waitcnt(0xC07F);
          __asm__ __volatile__("" ::: "memory");
          __builtin_amdgcn_s_barrier();
          __asm__ __volatile__("" ::: "memory");
#pragma unroll
          for (int h = 0; h < G; h++) mx[h] = fmaxf(fmaxf(red[h], red[G + h]), fmaxf(red[2 * G + h], red[3 * G + h]));
          const int nt = it.t1 - it.t0;
          for (int i = tid; i < nt; i += 256)
#pragma unroll
            for (int h = 0; h < G; h++) sc[i * G + h] = dexp(sc[i * G + h] - mx[h]);
          // the next iteration's barrier orders these writes before PV reads them
        }
      } else {
        // ---- PV: wave g = lane group g, rows r = 4 rd + g of the chunk -------------
        const int c = p - it.nch;
        const unsigned char* vb = reinterpret_cast<const unsigned char*>(buf);
#pragma unroll
        for (int rd = 0; rd < CT / 4; rd++) {
          const int r = rd * 4 + wave;
          const int t = it.T0 + c * CT + r;
          const bool ok = t >= it.t0 && t < it.t1;
          float vv[DPL];
          if constexpr (DPL == 2) {
            const h2 hv = *reinterpret_cast<const h2*>(vb + r * HD * 2 + lane * DPL * 2);
            vv[0] = ok ? (float)hv[0] : 0.0f;
            vv[1] = ok ? (float)hv[1] : 0.0f;
          } else {
            const h4 hv = *reinterpret_cast<const h4*>(vb + r * HD * 2 + lane * DPL * 2);
#pragma unroll
            for (int e = 0; e < 4; e++) vv[e] = ok ? (float)hv[e] : 0.0f;
          }
          const float* ps = sc + (size_t)(ok ? t - it.t0 : 0) * G;
#pragma unroll
          for (int h = 0; h < G; h++) {
            const float pr = ok ? ps[h] : 0.0f;
            l[h] = l[h] + pr;
#pragma unroll
            for (int d = 0; d < DPL; d++) o[h][d] = __builtin_fmaf(pr, vv[d], o[h][d]);
          }
        }
      }
    }
    // ---- combine the four groups ((0+1)+(2+3)) and write the partial ------------
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();  // every read of the ring is done: it becomes the combine buffer
#pragma unroll
    for (int h = 0; h < G; h++) {
#pragma unroll
      for (int d = 0; d < DPL; d++) comb[(wave * G + h) * HD + lane * DPL + d] = o[h][d];
      if (lane == 0) red[wave * G + h] = l[h];
    }
    __syncthreads();
    if constexpr (DIRECT) {
      // The lane's whole visible range is this one split: k_attn_merge's sums
      // for one partial (w = exp(m - M) with M = m, L = fmaf(l, w, 0),
      // O = fmaf(o, w, 0) / L) and its quantisation for the output projection,
      // eight dims per thread, the four threads of a 32-dim block adjacent.
      const int nb = n_kv * G * HD / 32;
      for (int e = tid; e < G * HD / 8; e += 256) {
        const int h = e / (HD / 8), d8 = (e % (HD / 8)) * 8;
        float m = mx[0];
#pragma unroll
        for (int k = 1; k < G; k++)
          if (h == k) m = mx[k];
        const float* lc = red;
        const float w = dexp(m - m);
        const float L = __builtin_fmaf((lc[h] + lc[G + h]) + (lc[2 * G + h] + lc[3 * G + h]), w, 0.0f);
        float O[8];
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const int c = h * HD + d8 + i;
          const float o = (comb[0 * G * HD + c] + comb[1 * G * HD + c]) + (comb[2 * G * HD + c] + comb[3 * G * HD + c]);
          O[i] = __builtin_fmaf(o, w, 0.0f) / L;
          a = fmaxf(a, fabsf(O[i]));
        }
        a = fmaxf(a, xor_lane<1>(a));
        a = fmaxf(a, xor_lane<2>(a));
        const float dq = act_scale(a);
        const float id = (dq != 0.0f) ? 1.0f / dq : 0.0f;
        const int b = it.b;
        const int kcol0 = (it.kvh * G + h) * HD + d8;
        const int blk = kcol0 >> 5, g8 = (kcol0 & 31) >> 3;
        h8 qv;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          float v = __builtin_rintf(O[i] * id);
          v = fminf(127.0f, fmaxf(-127.0f, v));
          qv[i] = (_Float16)(v * dq);
        }
        *reinterpret_cast<h8*>(ao.q + ((((size_t)(b >> 4) * nb + blk) * 4 + g8) * 16 + (b & 15)) * 8) = qv;
        if (g8 == 0) ao.s[(size_t)blk * ao.mpad + b] = dq;
      }
      __syncthreads();  // the combine buffer is read before the next item's DMA refills the ring
      continue;
    }
    float* rec = part + (size_t)it.idx * G * PF;
    for (int e = tid; e < G * HD / 4; e += 256) {
      const int h = e / (HD / 4), d4 = (e % (HD / 4)) * 4;
      f4 out;
#pragma unroll
      for (int i = 0; i < 4; i++)
        out[i] = (comb[(0 * G + h) * HD + d4 + i] + comb[(1 * G + h) * HD + d4 + i]) +
                 (comb[(2 * G + h) * HD + d4 + i] + comb[(3 * G + h) * HD + d4 + i]);
      *reinterpret_cast<f4*>(rec + h * PF + d4) = out;
    }
    if (tid < G) {
      const float* lc = red;
      float m = mx[0];
#pragma unroll
      for (int h = 1; h < G; h++)
        if (tid == h) m = mx[h];
      rec[tid * PF + HD] = m;
      rec[tid * PF + HD + 1] = (lc[tid] + lc[G + tid]) + (lc[2 * G + tid] + lc[3 * G + tid]);
    }
    __syncthreads();  // the combine buffer is read before the next item's DMA refills the ring
  }
}

// Ring depth: deeper rings keep more rows in flight per wave (fewer waves fit).
#define RSTR_ATTN_RING 3

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

// One split-kernel instantiation: its LDS bytes and its resident grid (one
// wave per workgroup, every wave resident, never more waves than items).
template <int HD, int G, int LPT>
struct AttnSplit {
  // Ring depth of the one-wave kernel: RB, or RB - 1 where the shallower
  // ring lets more waves reside on a CU (instantiations whose LDS, not their
  // registers, bound the occupancy: config3's Qwen3 geometry at split 256
  // goes from 10 to 12 waves per CU, 3.85-3.89 -> 3.75-3.79 ms/step; the
  // Llama geometry is register-bound at 8 waves either way and keeps RB).
  static constexpr int RB = RSTR_ATTN_RING;
  static constexpr int RBS = RSTR_ATTN_RING - 1;
  static size_t lds(const AttnGeom& g, int rb) {
    return (size_t)rb * 16 * (HD / 8) * 16 + (size_t)((G * HD * 4 + 1023) / 1024) * 1024 +
           sizeof(float) * G * g.split;
  }
  // whole-page chunks: page_size a power of two and a multiple of 16
  static bool pg16(const AttnGeom& g) { return g.page_size % 16 == 0 && (g.page_size & (g.page_size - 1)) == 0; }
  static decltype(&k_attn_split<HD, G, LPT, true, RB>) kernel(const AttnGeom& g, int rb) {
    if (rb == RBS) return pg16(g) ? k_attn_split<HD, G, LPT, true, RBS> : k_attn_split<HD, G, LPT, false, RBS>;
    return pg16(g) ? k_attn_split<HD, G, LPT, true, RB> : k_attn_split<HD, G, LPT, false, RB>;
  }
  static int waves_per_cu(const AttnGeom& g, int rb) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel(g, rb), 64, lds(g, rb)) != hipSuccess) return 0;
    return n;
  }
  static int ring(const AttnGeom& g) { return waves_per_cu(g, RBS) > waves_per_cu(g, RB) ? RBS : RB; }
  // Few-item launches (k_attn_split_wg, one 4-wave workgroup per item): head
  // dim 128 or 256, whole-page chunks, and a largest work list that fits in
  // two rounds of resident workgroups.  Its ring is 32 KB deep.
  static constexpr bool kWG = HD == 128 || HD == 256;
  static constexpr int RBW = HD == 128 ? 8 : 4;
  static size_t lds_wg(const AttnGeom& g) {
    return (size_t)RBW * 16 * (HD / 8) * 16 + sizeof(float) * (G * (4 + (size_t)g.split) + (G + 1) * HD);
  }
  template <bool QKV = false>
  static int wg_capacity(const AttnGeom& g) {
    if constexpr (!kWG) {
      return 0;
    } else {
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_attn_split_wg<HD, G, RBW, QKV>, 256, lds_wg(g)) !=
          hipSuccess)
        return 0;
      return device_cus() * n;
    }
  }
  // The QKV form only where the whole work list is one round of resident
  // workgroups: its per-item prologue (the item's q from the projection
  // slices) sits on each item's path, so a second round pays it twice.
  // Measured: one lane of Llama-3-8B 2.43 -> 2.385 ms/step and config1
  // 0.761 -> 0.753 (one round), config2 0.794 -> 0.802 (two rounds).
  template <bool QKV = false>
  static bool use_wg(const AttnGeom& g, int max_items) {
    if (!kWG || !pg16(g)) return false;
    const int cap = wg_capacity<QKV>(g);
    return cap > 0 && max_items <= (QKV ? 1 : 2) * cap;
  }
  static int grid(const AttnGeom& g, int max_items) {
    if (use_wg(g, max_items)) return std::max(1, std::min(wg_capacity(g), max_items));
    int n = waves_per_cu(g, ring(g));
    if (n <= 0) n = 2;
    return std::max(1, std::min(device_cus() * n, max_items));
  }
  static void launch(hipStream_t st, const AttnGeom& g, const float* q, const uint16_t* kp,
                     const uint16_t* vp, const int32_t* pt, int32_t* tab, float* part,
                     int max_items, const AttnOut* out) {
    const int R = grid(g, max_items);
    const int32_t* n_items = tab + 4 * g.batch;  // base[batch]
    int* ctr = tab + attn_ctl_offset(g.batch);
    const int4* items = reinterpret_cast<const int4*>(tab + attn_items_offset(g.batch));
    const int shift = pg16(g) ? __builtin_ctz((unsigned)g.page_size) : 0;
    if constexpr (kWG) {
      if (use_wg(g, max_items)) {
        if (out)
          hipLaunchKernelGGL((k_attn_split_wg<HD, G, RBW, false, true>), dim3(R), dim3(256), lds_wg(g), st, g.n_kv,
                             g.page_size, shift, g.pps, g.scale, q, kp, vp, pt, n_items, items, part, AttnQkv{},
                             *out);
        else
          hipLaunchKernelGGL((k_attn_split_wg<HD, G, RBW>), dim3(R), dim3(256), lds_wg(g), st, g.n_kv, g.page_size,
                             shift, g.pps, g.scale, q, kp, vp, pt, n_items, items, part, AttnQkv{}, AttnOut{});
        return;
      }
    }
    const int rb = ring(g);
    hipLaunchKernelGGL(kernel(g, rb), dim3(R), dim3(64), lds(g, rb), st, g.n_kv, g.page_size, shift, g.pps, g.scale,
                       q, kp, vp, pt, n_items, items, ctr, part);
  }
  // the few-item kernel with the qkv post-processing in its prologue
  static bool launch_qkv(hipStream_t st, const AttnGeom& g, const AttnQkv& qk, const int32_t* pt, int32_t* tab,
                         float* part, int max_items, const AttnOut* out) {
    if constexpr (kWG) {
      if (!use_wg<true>(g, max_items)) return false;
      const int R = std::max(1, std::min(wg_capacity<true>(g), max_items));
      const int32_t* n_items = tab + 4 * g.batch;
      const int4* items = reinterpret_cast<const int4*>(tab + attn_items_offset(g.batch));
      const int shift = __builtin_ctz((unsigned)g.page_size);
      if (out)
        hipLaunchKernelGGL((k_attn_split_wg<HD, G, RBW, true, true>), dim3(R), dim3(256), lds_wg(g), st, g.n_kv,
                           g.page_size, shift, g.pps, g.scale, nullptr, qk.kpages, qk.vpages, pt, n_items, items,
                           part, qk, *out);
      else
        hipLaunchKernelGGL((k_attn_split_wg<HD, G, RBW, true>), dim3(R), dim3(256), lds_wg(g), st, g.n_kv,
                           g.page_size, shift, g.pps, g.scale, nullptr, qk.kpages, qk.vpages, pt, n_items, items,
                           part, qk, AttnOut{});
      return true;
    } else {
      return false;
    }
  }
};

// Dispatch over the supported (head dim, GQA group) pairs with their QK lane
// counts; OP(HD, G, LPT) must return.
#define RSTR_ATTN_DISPATCH(g, OP)                                                          \
  do {                                                                                     \
    const int G_ = (g).n_q / (g).n_kv;                                                     \
    if ((g).hd == 64 && G_ == 1) OP(64, 1, 4);                                             \
    if ((g).hd == 64 && G_ == 2) OP(64, 2, 4);                                             \
    if ((g).hd == 64 && G_ == 4) OP(64, 4, 4);                                             \
    if ((g).hd == 64 && G_ == 8) OP(64, 8, 4);                                             \
    if ((g).hd == 128 && G_ == 1) OP(128, 1, 4);                                           \
    if ((g).hd == 128 && G_ == 2) OP(128, 2, 4);                                           \
    if ((g).hd == 128 && G_ == 4) OP(128, 4, 8);                                           \
    if ((g).hd == 128 && G_ == 8) OP(128, 8, 8);                                           \
    if ((g).hd == 256 && G_ == 1) OP(256, 1, 4);                                           \
    if ((g).hd == 256 && G_ == 2) OP(256, 2, 8);                                           \
    if ((g).hd == 256 && G_ == 4) OP(256, 4, 8);                                           \
    if ((g).hd == 256 && G_ == 8) OP(256, 8, 16);                                          \
  } while (0)

int attn_grid(const AttnGeom& g, int max_items) {
#define RSTR_AG(HD_, G_, L_) return AttnSplit<HD_, G_, L_>::grid(g, max_items)
  RSTR_ATTN_DISPATCH(g, RSTR_AG);
#undef RSTR_AG
  return 0;
}

size_t attn_tab_words(const AttnGeom& g, int max_items) {
  if (attn_grid(g, max_items) <= 0) return 0;
  return attn_items_offset(g.batch) + (size_t)4 * max_items;
}

hipError_t launch_attn_split(hipStream_t st, const AttnGeom& g, const float* q,
                             const uint16_t* kpages, const uint16_t* vpages,
                             const int32_t* page_table, int32_t* lane_tab, float* part,
                             int max_items, const AttnOut* out) {
  if (out && !attn_direct_out(g, max_items)) return hipErrorInvalidValue;
#define RSTR_AL(HD_, G_, L_)                                                                                 \
  {                                                                                                          \
    AttnSplit<HD_, G_, L_>::launch(st, g, q, kpages, vpages, page_table, lane_tab, part, max_items, out); \
    return hipGetLastError();                                                                                \
  }
  RSTR_ATTN_DISPATCH(g, RSTR_AL);
#undef RSTR_AL
  return hipErrorInvalidValue;
}

bool attn_direct_out(const AttnGeom& g, int max_items) {
#define RSTR_AD(HD_, G_, L_) return AttnSplit<HD_, G_, L_>::use_wg(g, max_items)
  RSTR_ATTN_DISPATCH(g, RSTR_AD);
#undef RSTR_AD
  return false;
}

bool attn_fuses_qkv(const AttnGeom& g, int max_items) {
#define RSTR_AF(HD_, G_, L_)                                                                 \
  return AttnSplit<HD_, G_, L_>::use_wg(g, max_items) && AttnSplit<HD_, G_, L_>::template use_wg<true>(g, max_items)
  RSTR_ATTN_DISPATCH(g, RSTR_AF);
#undef RSTR_AF
  return false;
}

hipError_t launch_attn_split_qkv(hipStream_t st, const AttnGeom& g, const AttnQkv& qk,
                                 const int32_t* page_table, int32_t* lane_tab, float* part, int max_items,
                                 const AttnOut* out) {
  if (g.hd > 256 || g.hd % 4) return hipErrorInvalidValue;
#define RSTR_AQ(HD_, G_, L_)                                                                                 \
  {                                                                                                         \
    if (!AttnSplit<HD_, G_, L_>::launch_qkv(st, g, qk, page_table, lane_tab, part, max_items, out))          \
      return hipErrorInvalidValue;                                                                          \
    return hipGetLastError();                                                                               \
  }
  RSTR_ATTN_DISPATCH(g, RSTR_AQ);
#undef RSTR_AQ
  return hipErrorInvalidValue;
}

// Merge splits of one (lane, q head) in split order and quantise the row
// block for the output projection: w = exp(m_k - M), L = fmaf(l_k, w, L),
// O = fmaf(o_k, w, O), out = O / L.  Empty routes output 0.
template <int HD>
__global__ __launch_bounds__(64) void k_attn_merge(int batch, int n_q, int n_kv,
                                                   const int32_t* __restrict__ lengths,
                                                   int32_t* __restrict__ tab,
                                                   const float* __restrict__ part,
                                                   float* __restrict__ out_f32,
                                                   _Float16* __restrict__ Q, float* __restrict__ S,
                                                   int mpad) {
  constexpr int DPL = HD / 64;
  const int lane = threadIdx.x;
  const int b = blockIdx.x / n_q, h = blockIdx.x % n_q;
  const int G = n_q / n_kv;
  // the split kernel of this layer has finished: re-arm its claim counter
  // for the next split over this table
  if (blockIdx.x == 0 && lane == 0) tab[attn_ctl_offset(batch)] = tab[attn_ctl_offset(batch) + 1];
  const int ns = tab[2 * batch + b];
  const int base = tab[3 * batch + b] + (h / G) * ns;
  const int hl = h % G;
  const int len = lengths[b];
  float O[DPL];
#pragma unroll
  for (int d = 0; d < DPL; d++) O[d] = 0.0f;
  if (len > 0 && ns > 0) {
    // Split partials, in split order; every load of a batch is issued before
    // its first use.  First batch: the o of splits 0..15 with the m and l of
    // split `lane` (and the m of splits lane+64, ... for the maximum); then 16
    // splits' o per batch.  w_k = exp(m_k - M) is computed once by lane k mod 64
    // and read from that lane (same value, same order of the fmas below).
    constexpr int C = 16;
    const int stride = G * attn_part_floats(HD);
    const float* pb = part + (size_t)base * stride + hl * attn_part_floats(HD);
    float ok[C][DPL];
#pragma unroll
    for (int j = 0; j < C; j++) {
      const float* pr = pb + (size_t)min(j, ns - 1) * stride;
#pragma unroll
      for (int d = 0; d < DPL; d++) ok[j][d] = pr[lane * DPL + d];
    }
    const float* p0 = pb + (size_t)min(lane, ns - 1) * stride;
    const float m0 = p0[HD], l0 = p0[HD + 1];
    float M = m0;
    for (int kk = lane + 64; kk < ns; kk += 64) M = fmaxf(M, pb[(size_t)kk * stride + HD]);
    M = wave_max(M);
    float L = 0.0f;
    for (int g0 = 0; g0 < ns; g0 += 64) {
      float wl, ll;
      if (g0 == 0) {
        wl = dexp(m0 - M);
        ll = l0;
      } else {
        const float* pk = pb + (size_t)min(g0 + lane, ns - 1) * stride;
        wl = dexp(pk[HD] - M);
        ll = pk[HD + 1];
      }
      const int gn = min(64, ns - g0);
      for (int c0 = 0; c0 < gn; c0 += C) {
        if (g0 + c0 > 0) {
#pragma unroll
          for (int j = 0; j < C; j++) {
            const float* pr = pb + (size_t)min(g0 + c0 + j, ns - 1) * stride;
#pragma unroll
            for (int d = 0; d < DPL; d++) ok[j][d] = pr[lane * DPL + d];
          }
        }
#pragma unroll
        for (int j = 0; j < C; j++) {
          if (c0 + j < gn) {
            const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), c0 + j));
            const float lk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ll), c0 + j));
            L = __builtin_fmaf(lk, w, L);
#pragma unroll
            for (int d = 0; d < DPL; d++) O[d] = __builtin_fmaf(ok[j][d], w, O[d]);
          }
        }
      }
    }
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
    const float dq = act_scale(a);
    const float id = (dq != 0.0f) ? 1.0f / dq : 0.0f;
    const int qd = n_q * HD, nb = qd >> 5;
#pragma unroll
    for (int d = 0; d < DPL; d++) {
      const int kcol = h * HD + lane * DPL + d;
      float v = __builtin_rintf(O[d] * id);
      v = fminf(127.0f, fmaxf(-127.0f, v));
      const int blk = kcol >> 5, g = (kcol & 31) >> 3, s = kcol & 7;
      Q[((((size_t)(b >> 4) * nb + blk) * 4 + g) * 16 + (b & 15)) * 8 + s] = (_Float16)(v * dq);
      if ((kcol & 31) == 0) S[(size_t)blk * mpad + b] = dq;
    }
  }
}

// The same merge with one wave per (lane, q head, 64 dims), one dim per lane,
// for grids of under two (lane, head) waves per SIMD, where the merge is
// latency bound: a wave holds one value per split and
// loads C splits at once (64 for head dim 256, 32 below), one dependent memory
// round trip per C splits instead of per 16.  Every dim's sums are the same
// fmaf chains in split order as above, and L, M and w are formed identically
// by the head's waves.
template <int HD>
__global__ __launch_bounds__(64) void k_attn_merge_wide(int batch, int n_q, int n_kv,
                                                   const int32_t* __restrict__ lengths,
                                                   int32_t* __restrict__ tab,
                                                   const float* __restrict__ part,
                                                   float* __restrict__ out_f32,
                                                   _Float16* __restrict__ Q, float* __restrict__ S,
                                                   int mpad) {
  constexpr int NQB = HD / 64;         // 64-dim blocks of a head, one wave each
  constexpr int C = HD >= 256 ? 64 : 32;  // splits loaded at once
  const int lane = threadIdx.x;
  const int bh = blockIdx.x / NQB, qb = blockIdx.x % NQB;
  const int b = bh / n_q, h = bh % n_q;
  const int G = n_q / n_kv;
  // the split kernel of this layer has finished: re-arm its claim counter
  // for the next split over this table
  if (blockIdx.x == 0 && lane == 0) tab[attn_ctl_offset(batch)] = tab[attn_ctl_offset(batch) + 1];
  const int ns = tab[2 * batch + b];
  const int base = tab[3 * batch + b] + (h / G) * ns;
  const int hl = h % G;
  const int len = lengths[b];
  const int dim = qb * 64 + lane;
  float O = 0.0f;
  if (len > 0 && ns > 0) {
    const int stride = G * attn_part_floats(HD);
    const float* pb = part + (size_t)base * stride + hl * attn_part_floats(HD);
    float ov[C];
#pragma unroll
    for (int j = 0; j < C; j++) ov[j] = pb[(size_t)min(j, ns - 1) * stride + dim];
    const float* p0 = pb + (size_t)min(lane, ns - 1) * stride;
    const float m0 = p0[HD], l0 = p0[HD + 1];
    float M = m0;
    for (int kk = lane + 64; kk < ns; kk += 64) M = fmaxf(M, pb[(size_t)kk * stride + HD]);
    M = wave_max(M);
    float L = 0.0f, wl = 0.0f, ll = 0.0f;
    for (int c0 = 0; c0 < ns; c0 += C) {
      // w_k = exp(m_k - M) by lane k mod 64, read from that lane
      if (c0 == 0) {
        wl = dexp(m0 - M);
        ll = l0;
      } else if (c0 % 64 == 0) {
        const float* pk = pb + (size_t)min(c0 + lane, ns - 1) * stride;
        wl = dexp(pk[HD] - M);
        ll = pk[HD + 1];
      }
      if (c0 > 0) {
#pragma unroll
        for (int j = 0; j < C; j++) ov[j] = pb[(size_t)min(c0 + j, ns - 1) * stride + dim];
      }
      const int gn = min(C, ns - c0), l0off = c0 % 64;
#pragma unroll
      for (int j = 0; j < C; j++) {
        if (j < gn) {
          const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), l0off + j));
          const float lk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ll), l0off + j));
          L = __builtin_fmaf(lk, w, L);
          O = __builtin_fmaf(ov[j], w, O);
        }
      }
    }
    O = O / L;
  }
  if (out_f32) out_f32[((size_t)b * n_q + h) * HD + dim] = O;
  if (Q) {
    // 32-dim blocks: 32 lanes per block
    float a = fabsf(O);
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) a = fmaxf(a, __shfl_xor(a, m, 64));
    const float dq = act_scale(a);
    const float id = (dq != 0.0f) ? 1.0f / dq : 0.0f;
    const int qd = n_q * HD, nb = qd >> 5;
    const int kcol = h * HD + dim;
    float v = __builtin_rintf(O * id);
    v = fminf(127.0f, fmaxf(-127.0f, v));
    const int blk = kcol >> 5, g = (kcol & 31) >> 3, s = kcol & 7;
    Q[((((size_t)(b >> 4) * nb + blk) * 4 + g) * 16 + (b & 15)) * 8 + s] = (_Float16)(v * dq);
    if ((kcol & 31) == 0) S[(size_t)blk * mpad + b] = dq;
  }
}

hipError_t launch_attn_merge(hipStream_t st, const AttnGeom& g, const int32_t* lengths,
                             int32_t* lane_tab, const float* part, float* out_f32,
                             ActBuf* out_q) {
  _Float16* Q = out_q ? out_q->q : nullptr;
  float* S = out_q ? out_q->s : nullptr;
  int mpad = out_q ? out_q->mpad : 0;
  // under two (lane, head) waves per SIMD the merge is latency bound: spread
  // each head over HD/64 waves; above, one wave per head does less work per
  // output
  const bool wide = g.batch * g.n_q < 2048;
  dim3 grid(g.batch * g.n_q * (wide ? g.hd / 64 : 1));
#define RSTR_MERGE(HDV)                                                                                  \
  hipLaunchKernelGGL(wide ? k_attn_merge_wide<HDV> : k_attn_merge<HDV>, grid, dim3(64), 0, st, g.batch, \
                     g.n_q, g.n_kv, lengths, lane_tab, part, out_f32, Q, S, mpad)
  if (g.hd == 64)
    RSTR_MERGE(64);
  else if (g.hd == 128)
    RSTR_MERGE(128);
  else if (g.hd == 256)
    RSTR_MERGE(256);
  else
    return hipErrorInvalidValue;
#undef RSTR_MERGE
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

// The tail in two launches: S workgroups per row each reduce one segment of
// the row's logits to a (value, index) candidate, then one wave per row picks
// the winner among its S candidates and gathers the embedding row.  The
// winner does not depend on the order in which candidates are compared
// (arg_take is a total order), so splitting the row is exact; one workgroup
// per row left most of the GPU idle on small batches (16 rows x 262144
// logits: 57 us).
int argmax_segments(int rows, int vocab) {
  int s = (2048 + rows - 1) / std::max(rows, 1);
  s = std::min(s, std::max(1, vocab / 2048));
  return std::max(1, std::min(s, 64));
}

__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ logits, int vocab, int seg,
                                                     int32_t* __restrict__ cand) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int s = blockIdx.x, row = blockIdx.y, S = gridDim.x, tid = threadIdx.x;
  const int lo = min(vocab, s * seg), hi = min(vocab, lo + seg);
  const float* lr = logits + (size_t)row * vocab;
  float bv = 0.0f;
  int bi = INT_MAX;
  if ((vocab & 3) == 0) {
    // seg is a multiple of 4: float4 chunks, four loads in flight per thread
    const int c0 = lo >> 2, n4 = (hi - lo) >> 2;
    const f4* l4 = reinterpret_cast<const f4*>(lr) + c0;
    for (int cb = tid; cb < n4; cb += 4 * 256) {
      f4 v[4];
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = l4[min(cb + j * 256, n4 - 1)];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int c = cb + j * 256;
        if (c < n4) {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (arg_take(bv, bi, v[j][e], lo + 4 * c + e)) { bv = v[j][e]; bi = lo + 4 * c + e; }
        }
      }
    }
  } else {
    for (int i = lo + tid; i < hi; i += 256) {
      const float v = lr[i];
      if (arg_take(bv, bi, v, i)) { bv = v; bi = i; }
    }
  }
  sv[tid] = bv;
  si[tid] = bi;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w && arg_take(sv[tid], si[tid], sv[tid + w], si[tid + w])) {
      sv[tid] = sv[tid + w];
      si[tid] = si[tid + w];
    }
    __syncthreads();
  }
  if (tid == 0) {
    cand[((size_t)row * S + s) * 2] = __builtin_bit_cast(int32_t, sv[0]);
    cand[((size_t)row * S + s) * 2 + 1] = si[0];
  }
}

__global__ __launch_bounds__(64) void k_argmax_final(const int32_t* __restrict__ cand, int S,
                                                     const float* __restrict__ emb, int d,
                                                     int32_t* __restrict__ tok, float* __restrict__ r0) {
  const int row = blockIdx.x, lane = threadIdx.x;
  float bv = 0.0f;
  int bi = INT_MAX;
  if (lane < S) {
    bv = __builtin_bit_cast(float, cand[((size_t)row * S + lane) * 2]);
    bi = cand[((size_t)row * S + lane) * 2 + 1];
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (arg_take(bv, bi, ov, oi)) { bv = ov; bi = oi; }
  }
  const int t = bi;
  if (lane == 0) tok[row] = t;
  const float* er = emb + (size_t)t * d;
  float* rr = r0 + (size_t)row * d;
  if ((d & 3) == 0) {
    // 16-byte pieces, eight loads in flight per lane before their stores (a
    // load-then-store loop waits one memory round trip per 256 bytes of row:
    // 26 us for a 4096-wide row)
    const f4* e4 = reinterpret_cast<const f4*>(er);
    f4* r4 = reinterpret_cast<f4*>(rr);
    const int n4 = d >> 2;
    for (int i0 = lane; i0 < n4; i0 += 8 * 64) {
      f4 v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = e4[min(i0 + 64 * j, n4 - 1)];
#pragma unroll
      for (int j = 0; j < 8; j++)
        if (i0 + 64 * j < n4) r4[i0 + 64 * j] = v[j];
    }
  } else {
    for (int i = lane; i < d; i += 64) rr[i] = er[i];
  }
}

hipError_t launch_argmax_gather(hipStream_t st, const float* logits, int rows, int vocab,
                                const float* emb, int d, int32_t* tok, float* r0, int32_t* cand) {
  const int S = argmax_segments(rows, vocab);
  const int seg = ((vocab + S - 1) / S + 3) & ~3;
  hipLaunchKernelGGL(k_argmax_part, dim3(S, rows), dim3(256), 0, st, logits, vocab, seg, cand);
  hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(64), 0, st, cand, S, emb, d, tok, r0);
  return hipGetLastError();
}

__global__ void k_gather_rows(const float* __restrict__ emb, int d, const int32_t* __restrict__ lanes,
                              const int32_t* __restrict__ tokens, float* __restrict__ r0) {
  const int i = blockIdx.x;
  const float* er = emb + (size_t)tokens[i] * d;
  float* rr = r0 + (size_t)lanes[i] * d;
  if ((d & 3) == 0) {
    // 16-byte pieces, four loads in flight per thread before their stores
    const f4* e4 = reinterpret_cast<const f4*>(er);
    f4* r4 = reinterpret_cast<f4*>(rr);
    const int n4 = d >> 2, nt = blockDim.x;
    for (int k0 = threadIdx.x; k0 < n4; k0 += 4 * nt) {
      f4 v[4];
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = e4[min(k0 + nt * j, n4 - 1)];
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (k0 + nt * j < n4) r4[k0 + nt * j] = v[j];
    }
  } else {
    for (int k = threadIdx.x; k < d; k += blockDim.x) rr[k] = er[k];
  }
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

// Checkpoint tensors to f32 on the device (safetensors.clj:48-72 read-tensor-
// floats): F16 widens exactly, BF16 is the upper half of an f32 bit pattern.
__global__ void k_widen(int dtype, const void* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (dtype == 1) dst[i] = (float)static_cast<const _Float16*>(src)[i];
  else if (dtype == 2) dst[i] = __builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(src)[i] << 16);
  else dst[i] = static_cast<const float*>(src)[i];
}

hipError_t launch_widen(hipStream_t st, int dtype, const void* src, float* dst, int64_t n) {
  if (n <= 0) return hipSuccess;
  if (dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_widen, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dtype, src, dst, n);
  return hipGetLastError();
}

// Durable chunk transfer: token rows between the page pool and a dense payload
// in the portable layout (page_pool.clj:1111-1374; payload order of
// attention_state.clj:103-123: slab K then V, layer, token; a row is `ept`
// fp16).  One thread moves one 16-byte piece of one row of one slab-layer;
// consecutive threads take consecutive pieces of a row, so both sides are
// coalesced whatever the page table looks like.  Mode 0 gathers pool ->
// payload, mode 1 scatters an fp16 payload, mode 2 scatters an f32 payload
// rounded to fp16 (round to nearest even, Float/floatToFloat16).
template <int MODE>
__global__ __launch_bounds__(256) void k_chunk_move(uint16_t* const* __restrict__ slabs,
                                                    const int32_t* __restrict__ pages, int start,
                                                    int count, int page_size, int ept,
                                                    int64_t n_pieces, void* __restrict__ payload) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_pieces) return;
  const int pieces = ept >> 3;
  const int piece = (int)(i % pieces);
  const int64_t r = i / pieces;             // (slab-layer, token) row of the payload
  const int t = (int)(r % count);
  const int sl = (int)(r / count);
  const int logical = start + t;
  const int64_t phys = (int64_t)pages[logical / page_size] * page_size + logical % page_size;
  uint16_t* row = slabs[sl] + phys * ept + piece * 8;
  const int64_t off = r * ept + piece * 8;
  if constexpr (MODE == 0) {
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(payload) + off) = *reinterpret_cast<const u32x4*>(row);
  } else if constexpr (MODE == 1) {
    *reinterpret_cast<u32x4*>(row) = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(payload) + off);
  } else {
    const float* src = static_cast<const float*>(payload) + off;
    const f4 a = *reinterpret_cast<const f4*>(src);
    const f4 b = *reinterpret_cast<const f4*>(src + 4);
    h8 h;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      h[k] = (_Float16)a[k];
      h[4 + k] = (_Float16)b[k];
    }
    *reinterpret_cast<h8*>(row) = h;
  }
}

hipError_t launch_chunk_move(hipStream_t st, int mode, uint16_t** slabs, int nslabs, const int32_t* pages,
                             int start, int count, int page_size, int ept, void* payload) {
  if (count <= 0) return hipSuccess;
  if (ept % 8) return hipErrorInvalidValue;
  const int64_t n = (int64_t)nslabs * count * (ept / 8);
  const dim3 grid((unsigned)((n + 255) / 256));
  if (mode == 0)
    hipLaunchKernelGGL(k_chunk_move<0>, grid, dim3(256), 0, st, slabs, pages, start, count, page_size, ept, n, payload);
  else if (mode == 1)
    hipLaunchKernelGGL(k_chunk_move<1>, grid, dim3(256), 0, st, slabs, pages, start, count, page_size, ept, n, payload);
  else if (mode == 2)
    hipLaunchKernelGGL(k_chunk_move<2>, grid, dim3(256), 0, st, slabs, pages, start, count, page_size, ept, n, payload);
  else
    return hipErrorInvalidValue;
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

// ===========================================================================
// The allocation-free entry's staging: one array per GPU, held until the
// process ends.  Host code never passes `scratch` itself to a kernel (in host
// code the name stands for a host-side shadow); it uses the device address
// that static_scratch_address returns for the current device.
// ===========================================================================
namespace rstr {
static __device__ __align__(256) unsigned char scratch[RSTR_STATIC_SCRATCH_BYTES];

hipError_t static_scratch_address(void** ptr) {
  *ptr = nullptr;
  return hipGetSymbolAddress(ptr, HIP_SYMBOL(scratch));
}
}  // namespace rstr

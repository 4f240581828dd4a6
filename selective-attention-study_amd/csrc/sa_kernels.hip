// Selective Attention for MI355X (gfx950): selection scan, forward, chunked prefill, backward.
//
// Operator (reference src/selective_attention/kernels.py:61-83, docs/kernel.md:32-46):
//   L_h = s Q_h K_h^T (causal),  S = relu(L_0) on E <= j < r,  F[i,j] = sum_{r<i} S[r,j],
//   O_h = softmax(L_h - F) V_h.
//
// Kernels (all 256 threads = 4 wavefronts of 64; MFMA 32x32 tiles):
//   sel_colsum   head 0, one 32x32 (queries x keys) tile per step: column sums of S per
//                32-query block -> colsum[b][rb][j]
//   sel_scan     exclusive running sum of colsum over query blocks, seeded by the carried
//                per-key state -> carry[b][rb][j], state_out[b][j]
//   fwd          query-parallel. A wavefront owns 32 queries of G heads. Logit tiles are
//                built transposed (keys x queries) so each lane holds one query: the online
//                softmax row statistics stay in-lane; the selection's exclusive prefix over
//                queries is a DPP lane scan, made once per tile and shared by the G heads.
//                O^T = V^T P^T takes P straight from the accumulator registers.
//   bwd          key-parallel. A wavefront owns 32 keys of G heads and sweeps the query
//                tiles last to first. Tiles are (queries x keys), so the selection prefix F
//                and the suffix U = sum_h sum_{i>r} dz_h[i,j] run down registers. dK, dV
//                stay in registers; dQ goes through LDS and relaxed fp32 atomics. The head
//                group holding head 0 folds g = -gate*U into head 0's own dz; other groups
//                add their share of head 0's gradient with atomics.
//
// MFMA operand layouts used throughout (v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x2_f32):
//   C (32x32, 16 fp32 per lane): lane l holds column l%32, rows crow(i, l/32), i = 0..15,
//                                crow(i,h) = 8*(i/4) + 4*h + i%4.
//   A (32xK) / B (Kx32):         lane l holds row (A) / column (B) l%32 and K elements
//                                [KS*step + (KS/2)*h, +KS/2) with KS = 16 (bf16) or 2 (fp32).
// A C-layout tile fed back as a B operand keeps its registers in place; the matching A operand
// is then read with the C layout's row order (ld_perm).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

#include "sa.h"

namespace {

typedef __bf16 bf16_t;
typedef bf16_t bf16x8 __attribute__((__vector_size__(8 * sizeof(bf16_t))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int TILE = 32;              // tile edge and carry checkpoint spacing (queries)
constexpr int NTHREADS = 256;
constexpr int NWAVES = 4;
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ int crow(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Wavefront-local ordering of LDS traffic (writes by some lanes, reads by others).
__device__ __forceinline__ void lds_wave_sync() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------------------------
// Operand traits: bf16 storage -> bf16 MFMA; fp32 storage -> fp32 MFMA.

struct OpBF16 {
  typedef uint16_t elem;
  typedef bf16x8 frag;
  static constexpr int KS = 16;
  static constexpr int KPAD = 8;     // LDS row padding (elements) of [rows][D] tiles
  static constexpr int TPAD = 4;     // LDS row padding (elements) of [rows][32] tiles

  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag zero() {
    frag f;
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] = (bf16_t)0.f;
    return f;
  }
  // Row r of a row-major tile, K elements [16*s + 8*h, +8).
  static __device__ __forceinline__ frag ld_std(const elem* p, int64_t ld, int r, int h, int s) {
    return *reinterpret_cast<const frag*>(p + r * ld + s * 16 + 8 * h);
  }
  // Row r, K elements in C-layout row order for step s: [16s+4h, +4) and [16s+8+4h, +4).
  static __device__ __forceinline__ frag ld_perm(const elem* p, int64_t ld, int r, int h, int s) {
    const elem* base = p + r * ld + s * 16 + 4 * h;
    uint2 lo = *reinterpret_cast<const uint2*>(base);
    uint2 hi = *reinterpret_cast<const uint2*>(base + 8);
    uint4 u = make_uint4(lo.x, lo.y, hi.x, hi.y);
    return *reinterpret_cast<frag*>(&u);
  }
  // C-layout registers [8s, 8s+8) as an operand (round to nearest even).
  static __device__ __forceinline__ frag from_acc(const f32x16& c, int s) {
    frag f;
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] = (bf16_t)c[8 * s + t];
    return f;
  }
  // The rounding residual of from_acc: c - bf16(c), itself rounded. hi + lo carries about 16
  // significant bits, so a product taken on both keeps its sum close to fp32.
  static constexpr bool SPLIT = true;
  static __device__ __forceinline__ frag from_acc_lo(const f32x16& c, int s) {
    frag f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float x = c[8 * s + t];
      f[t] = (bf16_t)(x - (float)(bf16_t)x);
    }
    return f;
  }
  static __device__ __forceinline__ elem to_elem(float x) {
    bf16_t b = (bf16_t)x;
    return *reinterpret_cast<elem*>(&b);
  }
  static __device__ __forceinline__ elem to_elem_lo(float x) { return to_elem(x - to_float(to_elem(x))); }
  static __device__ __forceinline__ float to_float(elem x) {
    return __uint_as_float(((uint32_t)x) << 16);
  }
  static constexpr int acc_steps = 2;   // C-layout K steps over 32 rows
};

struct OpF32 {
  typedef float elem;
  typedef float frag;
  static constexpr int KS = 2;
  static constexpr int KPAD = 4;
  static constexpr int TPAD = 1;

  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag zero() { return 0.f; }
  static __device__ __forceinline__ frag ld_std(const elem* p, int64_t ld, int r, int h, int s) {
    return p[r * ld + 2 * s + h];
  }
  static __device__ __forceinline__ frag ld_perm(const elem* p, int64_t ld, int r, int h, int s) {
    return p[r * ld + crow(s, h)];
  }
  static __device__ __forceinline__ frag from_acc(const f32x16& c, int s) { return c[s]; }
  static constexpr bool SPLIT = false;   // fp32 operands are exact already
  static __device__ __forceinline__ frag from_acc_lo(const f32x16& c, int s) { return 0.f; }
  static __device__ __forceinline__ elem to_elem(float x) { return x; }
  static __device__ __forceinline__ elem to_elem_lo(float x) { return 0.f; }
  static __device__ __forceinline__ float to_float(elem x) { return x; }
  static constexpr int acc_steps = 16;
};

// Fragment read straight from global memory with a row bound (rows >= nrows read as zero).
template <class OP>
__device__ __forceinline__ typename OP::frag ld_std_bounded(const typename OP::elem* p, int64_t ld,
                                                            int r, int nrows, int h, int s) {
  if (r < nrows) return OP::ld_std(p, ld, r, h, s);
  return OP::zero();
}

// B operand of a key-contracted product taken from a row-major [keys][D] global matrix:
// lane holds rows key0 + KS*s + (KS/2)*h + t, column d. Rows >= nrows read as zero.
template <class OP>
__device__ __forceinline__ typename OP::frag ld_colgather(const typename OP::elem* p, int D, int key0,
                                                          int nrows, int d, int h, int s) {
  typename OP::frag f;
  if constexpr (OP::KS == 16) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      int r = key0 + 16 * s + 8 * h + t;
      uint16_t raw = (r < nrows) ? p[(int64_t)r * D + d] : (uint16_t)0;
      f[t] = *reinterpret_cast<bf16_t*>(&raw);
    }
  } else {
    int r = key0 + 2 * s + h;
    f = (r < nrows) ? p[(int64_t)r * D + d] : 0.f;
  }
  return f;
}

// ---------------------------------------------------------------------------------------------
// LDS staging (whole workgroup).

// [32 rows][COLS] tile from a row-major global matrix (row stride gld); rows >= nrows are zero.
template <typename E, int COLS, int SLD>
__device__ __forceinline__ void stage_rows(E* s, const E* g, int64_t gld, int row0, int nrows, int tid) {
  constexpr int EPC = 16 / sizeof(E);
  constexpr int CPR = COLS / EPC;
  constexpr int NCH = TILE * CPR;
  static_assert((SLD * sizeof(E)) % 16 == 0, "row stride must keep 16-byte alignment");
#pragma unroll
  for (int c = tid; c < NCH; c += NTHREADS) {
    const int r = c / CPR, cc = (c % CPR) * EPC;
    uint4 val = make_uint4(0u, 0u, 0u, 0u);
    if (row0 + r < nrows) val = *reinterpret_cast<const uint4*>(g + (int64_t)(row0 + r) * gld + cc);
    *reinterpret_cast<uint4*>(s + r * SLD + cc) = val;
  }
}

// [ROWS][32] tile: columns col0..col0+31 of a row-major global matrix (row stride gld, 16-byte
// aligned rows); columns >= ncols are zero.
template <typename E, int ROWS, int SLD>
__device__ __forceinline__ void stage_cols(E* s, const E* g, int64_t gld, int col0, int ncols, int tid) {
  constexpr int EPC = 16 / sizeof(E);
  constexpr int CPR = TILE / EPC;
  constexpr int NCH = ROWS * CPR;
#pragma unroll
  for (int c = tid; c < NCH; c += NTHREADS) {
    const int r = c / CPR, cc = (c % CPR) * EPC;
    const E* src = g + (int64_t)r * gld + col0 + cc;
    union { uint4 v; E e[EPC]; uint2 h[2]; } u;
    if (col0 + cc + EPC <= ncols) {
      u.v = *reinterpret_cast<const uint4*>(src);
    } else {
#pragma unroll
      for (int e = 0; e < EPC; ++e) u.e[e] = (col0 + cc + e < ncols) ? src[e] : (E)0;
    }
    E* dst = s + r * SLD + cc;
    if constexpr (sizeof(E) == 2) {
      static_assert((SLD * 2) % 8 == 0, "bf16 transposed tiles need 8-byte row alignment");
      reinterpret_cast<uint2*>(dst)[0] = u.h[0];
      reinterpret_cast<uint2*>(dst)[1] = u.h[1];
    } else {
#pragma unroll
      for (int e = 0; e < EPC; ++e) dst[e] = u.e[e];
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Lane scans (DPP) across the 32 lanes of each half-wavefront.

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_shift(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}

// Exclusive prefix sum over lanes 0..31 and, separately, 32..63.
__device__ __forceinline__ float excl_scan32(float x) {
  float s = x;
  s += dpp_shift<0x111, 0xF>(s);   // row_shr:1
  s += dpp_shift<0x112, 0xF>(s);   // row_shr:2
  s += dpp_shift<0x114, 0xF>(s);   // row_shr:4
  s += dpp_shift<0x118, 0xF>(s);   // row_shr:8
  s += dpp_shift<0x142, 0xA>(s);   // row_bcast:15 into rows 1 and 3
  return s - x;
}

// ---------------------------------------------------------------------------------------------
// Selection column sums: colsum[b][rb][j] = sum over the queries r of block rb (chunk-relative)
// of S[r, j]. One wavefront per key block; RB query blocks per workgroup row.

template <class OP, int D>
__global__ __launch_bounds__(NTHREADS) void sel_colsum_kernel(
    const typename OP::elem* __restrict__ q, const typename OP::elem* __restrict__ k,
    float* __restrict__ colsum, int H, int Tq, int Tk, int q_off, int exempt, float scale, int RB) {
  using elem = typename OP::elem;
  using frag = typename OP::frag;
  constexpr int NS = D / OP::KS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int NKT = (Tk + TILE - 1) / TILE;
  const int NBq = (Tq + TILE - 1) / TILE;
  const int kb = blockIdx.x * NWAVES + wave;
  if (kb >= NKT) return;
  const int b = blockIdx.z;
  const elem* q0 = q + (int64_t)b * H * Tq * D;
  const elem* k0 = k + (int64_t)b * H * Tk * D;
  const int j = kb * TILE + n;

  frag kf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) kf[s] = ld_std_bounded<OP>(k0, D, kb * TILE + n, Tk, h, s);

  const int rb_end = min(NBq, (int)(blockIdx.y + 1) * RB);
  for (int rb = blockIdx.y * RB; rb < rb_end; ++rb) {
    float cs = 0.f;
    // the tile holds a selectable pair only if some query is after the first key
    if (q_off + rb * TILE + TILE - 1 > kb * TILE) {
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < NS; ++s)
        acc = OP::mma(ld_std_bounded<OP>(q0, D, rb * TILE + n, Tq, h, s), kf[s], acc);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = rb * TILE + crow(i, h);
        const float sv = acc[i] * scale;
        const bool gate = (r < Tq) && (j >= exempt) && (j < q_off + r) && (sv > 0.f);
        cs += gate ? sv : 0.f;
      }
      cs += xor32(cs);
    }
    if (h == 0 && j < Tk) colsum[((int64_t)b * NBq + rb) * Tk + j] = cs;
  }
}

// carry[b][rb][j] = state_in[b][j] + sum_{rb' < rb} colsum[b][rb'][j] (in place);
// state_out[b][j] = the sum over all blocks. state_in is read for j < q_off only.
__global__ __launch_bounds__(NTHREADS) void sel_scan_kernel(
    float* __restrict__ carry, const float* state_in, float* state_out, int64_t state_ld,
    int NBq, int Tk, int q_off) {
  const int j = blockIdx.x * NTHREADS + threadIdx.x;
  const int b = blockIdx.y;
  if (j >= Tk) return;
  float run = (state_in != nullptr && j < q_off) ? state_in[(int64_t)b * state_ld + j] : 0.f;
  float* col = carry + (int64_t)b * NBq * Tk + j;
  for (int rb = 0; rb < NBq; ++rb) {
    const float c = col[(int64_t)rb * Tk];
    col[(int64_t)rb * Tk] = run;
    run += c;
  }
  state_out[(int64_t)b * state_ld + j] = run;
}

// ---------------------------------------------------------------------------------------------
// Forward. grid (ceil(NBq/4), nseq * H/G); wavefront w of block x owns query block
// (gridDim.x-1-x)*4 + w (heavy causal rows launch first) of heads [gi*G, gi*G+G).

template <class OP, int D, int G>
__global__ __launch_bounds__(NTHREADS) void fwd_kernel(
    const typename OP::elem* __restrict__ q, const typename OP::elem* __restrict__ k,
    const typename OP::elem* __restrict__ vt, const float* __restrict__ carry,
    float* __restrict__ out, float* __restrict__ rmax, float* __restrict__ rden,
    int H, int Tq, int Tk, int q_off, int64_t ldv, int exempt, float scale,
    int damp_mode, float train_len) {
  using elem = typename OP::elem;
  using frag = typename OP::frag;
  constexpr int NS = D / OP::KS;          // MFMA steps over D
  constexpr int DB = D / 32;              // 32-row blocks of D
  constexpr int LDK = D + OP::KPAD;
  constexpr int LDV = TILE + OP::TPAD;
  constexpr int AS = OP::acc_steps;

  __shared__ __attribute__((aligned(16))) elem sK[G + 1][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sVt[G][D * LDV];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int groups = H / G;
  const int b = blockIdx.y / groups, gi = blockIdx.y % groups;
  const int hd0 = gi * G;
  const bool has_h0 = (gi == 0);
  const int NBq = (Tq + TILE - 1) / TILE;
  const int NKT = (Tk + TILE - 1) / TILE;
  const int qsb = gridDim.x - 1 - blockIdx.x;
  const int rb = qsb * NWAVES + wave;
  const int q_rel = rb * TILE + n;
  const int q_abs = q_off + q_rel;
  const int64_t seq_row = (int64_t)b * H;   // row of head 0 of this sequence

  auto kt_end_of = [&](int rbw) {
    const int last = q_off + rbw * TILE + TILE - 1;
    return min(last / TILE + 1, NKT);
  };
  const int my_end = (rb < NBq) ? kt_end_of(rb) : 0;
  const int wg_end = kt_end_of(min(qsb * NWAVES + NWAVES - 1, NBq - 1));

  // Q fragments (B operand of K Q^T): lane holds query q_rel.
  frag qf[G][NS];
  frag q0f[NS];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const elem* qh = q + (seq_row + hd0 + g) * Tq * D;
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[g][s] = ld_std_bounded<OP>(qh, D, q_rel, Tq, h, s);
  }
  if (!has_h0) {
    const elem* qh = q + seq_row * Tq * D;
#pragma unroll
    for (int s = 0; s < NS; ++s) q0f[s] = ld_std_bounded<OP>(qh, D, q_rel, Tq, h, s);
  }

  float m[G], l[G];
  f32x16 o[G][DB];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[g][db] = zero16();
  }

  const float sl2 = scale * LOG2E;
  float damp = 1.f;
  if (damp_mode != 0) {
    damp = fminf(1.f, train_len / (float)(q_abs + 1));
    if (damp_mode == 2) damp = sqrtf(damp);
  }
  const float* carry_row = carry + ((int64_t)b * NBq + min(rb, NBq - 1)) * Tk;

  for (int kt = 0; kt < wg_end; ++kt) {
    const int kbase = kt * TILE;
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      stage_rows<elem, D, LDK>(sK[g], k + (seq_row + hd0 + g) * Tk * D, D, kbase, Tk, tid);
      stage_cols<elem, D, LDV>(sVt[g], vt + (seq_row + hd0 + g) * D * ldv, ldv, kbase, Tk, tid);
    }
    if (!has_h0) stage_rows<elem, D, LDK>(sK[G], k + seq_row * Tk * D, D, kbase, Tk, tid);
    __syncthreads();
    if (kt >= my_end) continue;

    const bool diag = (kbase + TILE - 1 > q_off + rb * TILE) || (kbase + TILE > Tk);

    // head 0 logits (keys x queries) -> selection S -> F (log2 units)
    f32x16 l0 = zero16();
    {
      const elem* k0s = has_h0 ? sK[0] : sK[G];
#pragma unroll
      for (int s = 0; s < NS; ++s)
        l0 = OP::mma(OP::ld_std(k0s, LDK, n, h, s), has_h0 ? qf[0][s] : q0f[s], l0);
    }
    f32x16 fs;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = kbase + crow(i, h);
      const float sv = l0[i] * scale;
      const bool gate = (j >= exempt) && (j < q_abs) && (sv > 0.f);
      const float sel = gate ? sv : 0.f;
      const float cj = (j < Tk) ? carry_row[j] : 0.f;
      fs[i] = (cj + excl_scan32(sel)) * (LOG2E * damp);
    }

#pragma unroll
    for (int g = 0; g < G; ++g) {
      f32x16 lg;
      if (g == 0 && has_h0) {
        lg = l0;
      } else {
        lg = zero16();
#pragma unroll
        for (int s = 0; s < NS; ++s) lg = OP::mma(OP::ld_std(sK[g], LDK, n, h, s), qf[g][s], lg);
      }
      float zmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float z = lg[i] * sl2 - fs[i];
        if (diag) {
          const int j = kbase + crow(i, h);
          if (j > q_abs || j >= Tk) z = -INFINITY;
        }
        lg[i] = z;
        zmax = fmaxf(zmax, z);
      }
      zmax = fmaxf(zmax, xor32(zmax));
      const float m_new = fmaxf(m[g], zmax);
      const float alpha = fast_exp2(m[g] - m_new);
      m[g] = m_new;
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float p = fast_exp2(lg[i] - m_new);
        lg[i] = p;
        psum += p;
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[g][db][i] *= alpha;
#pragma unroll
        for (int s = 0; s < AS; ++s)
          o[g][db] = OP::mma(OP::ld_perm(sVt[g], LDV, db * 32 + n, h, s), OP::from_acc(lg, s), o[g][db]);
      }
    }
  }

  if (rb >= NBq || q_rel >= Tq) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float ltot = l[g] + xor32(l[g]);
    const float inv = 1.f / ltot;
    const int64_t row = (seq_row + hd0 + g) * Tq + q_rel;
    float* orow = out + row * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        float4 v4 = make_float4(o[g][db][4 * a] * inv, o[g][db][4 * a + 1] * inv,
                                o[g][db][4 * a + 2] * inv, o[g][db][4 * a + 3] * inv);
        *reinterpret_cast<float4*>(orow + db * 32 + 8 * a + 4 * h) = v4;
      }
    }
    if (h == 0) {
      rmax[row] = m[g];
      rden[row] = ltot;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward preparation: lse = rmax + log2(rden), dbar = rowsum(dO * O), and the transposed
// copies Q^T, dO^T (R, D, ldt). One thread per row for the statistics; transposes by tiles.

template <class OP, int D>
__global__ __launch_bounds__(NTHREADS) void bwd_rowstats_kernel(
    const typename OP::elem* __restrict__ dout, const float* __restrict__ out,
    const float* __restrict__ rmax, const float* __restrict__ rden,
    float* __restrict__ lse, float* __restrict__ dbar, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * NTHREADS + threadIdx.x;
  if (r >= rows) return;
  const typename OP::elem* dr = dout + r * D;
  const float* orow = out + r * D;
  float acc = 0.f;
#pragma unroll 8
  for (int d = 0; d < D; ++d) acc += OP::to_float(dr[d]) * orow[d];
  dbar[r] = acc;
  lse[r] = rmax[r] + __log2f(rden[r]);
}

// in (R, T, D) -> outT (R, D, ldt); a workgroup moves a [64 t][D] slab through LDS.
template <typename E, int D>
__global__ __launch_bounds__(NTHREADS) void transpose_kernel(const E* __restrict__ in, E* __restrict__ outT,
                                                             int T, int64_t ldt) {
  __shared__ E tile[64][D + 1];
  const int64_t r = blockIdx.y;
  const int t0 = blockIdx.x * 64;
  const E* src = in + r * T * D;
  for (int c = threadIdx.x; c < 64 * D; c += NTHREADS) {
    const int tt = c / D, d = c % D;
    tile[tt][d] = (t0 + tt < T) ? src[(int64_t)(t0 + tt) * D + d] : (E)0;
  }
  __syncthreads();
  E* dst = outT + r * D * ldt;
  for (int c = threadIdx.x; c < 64 * D; c += NTHREADS) {
    const int d = c / 64, tt = c % 64;
    if (t0 + tt < ldt) dst[(int64_t)d * ldt + t0 + tt] = tile[tt][d];
  }
}

__global__ __launch_bounds__(NTHREADS) void fill_zero_kernel(float4* __restrict__ p, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * NTHREADS + threadIdx.x; i < n4; i += (int64_t)gridDim.x * NTHREADS)
    p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

// ---------------------------------------------------------------------------------------------
// Backward main kernel. grid (ceil(T/128), nseq * H/G); wavefront w owns keys
// [x*128 + 32w, +32) of heads [gi*G, gi*G+G).

template <class OP, int D, int G>
__global__ __launch_bounds__(NTHREADS) void bwd_kernel(
    const typename OP::elem* __restrict__ q, const typename OP::elem* __restrict__ k,
    const typename OP::elem* __restrict__ v, const typename OP::elem* __restrict__ qt,
    const typename OP::elem* __restrict__ dout, const typename OP::elem* __restrict__ dot,
    const float* __restrict__ lse, const float* __restrict__ dbar, const float* __restrict__ carry,
    float* __restrict__ dq, float* __restrict__ dk, float* __restrict__ dv, float* __restrict__ dk0x,
    int H, int T, int64_t ldt, int exempt, float scale) {
  using elem = typename OP::elem;
  using frag = typename OP::frag;
  constexpr int NS = D / OP::KS;
  constexpr int DB = D / 32;
  constexpr int LDK = D + OP::KPAD;
  constexpr int LDV = TILE + OP::TPAD;
  constexpr int LDZ = TILE + OP::KPAD;
  constexpr int AS = OP::acc_steps;
  constexpr int NH = G + 1;   // staged heads: the group, then head 0 when outside the group

  __shared__ __attribute__((aligned(16))) elem sQ[NH][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sQt[NH][D * LDV];
  __shared__ __attribute__((aligned(16))) elem sdO[G][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sdOt[G][D * LDV];
  __shared__ __attribute__((aligned(16))) float sLse[G][TILE];
  __shared__ __attribute__((aligned(16))) float sDb[G][TILE];
  __shared__ __attribute__((aligned(16))) elem sZ[NWAVES][TILE * LDZ];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int groups = H / G;
  const int b = blockIdx.y / groups, gi = blockIdx.y % groups;
  const int hd0 = gi * G;
  const bool has_h0 = (gi == 0);
  const int NB = (T + TILE - 1) / TILE;
  const int key0 = blockIdx.x * (NWAVES * TILE) + wave * TILE;
  const int j = key0 + n;
  const int64_t seq_row = (int64_t)b * H;
  elem* zs = sZ[wave];

  // Key-side operands in registers.
  frag kf[G][NS], vf[G][NS], ktf[G][DB][AS];
  frag k0f[NS], k0tf[DB][AS];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const elem* kh = k + (seq_row + hd0 + g) * T * D;
    const elem* vh = v + (seq_row + hd0 + g) * T * D;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      kf[g][s] = ld_std_bounded<OP>(kh, D, j, T, h, s);
      vf[g][s] = ld_std_bounded<OP>(vh, D, j, T, h, s);
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s) ktf[g][db][s] = ld_colgather<OP>(kh, D, key0, T, db * 32 + n, h, s);
  }
  if (!has_h0) {
    const elem* kh = k + seq_row * T * D;
#pragma unroll
    for (int s = 0; s < NS; ++s) k0f[s] = ld_std_bounded<OP>(kh, D, j, T, h, s);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s) k0tf[db][s] = ld_colgather<OP>(kh, D, key0, T, db * 32 + n, h, s);
  }

  f32x16 dkt[G][DB], dvt[G][DB], dk0t[DB];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      dkt[g][db] = zero16();
      dvt[g][db] = zero16();
    }
#pragma unroll
  for (int db = 0; db < DB; ++db) dk0t[db] = zero16();

  float ucarry = 0.f;
  const float sl2 = scale * LOG2E;
  const int qb_lo = (blockIdx.x * NWAVES * TILE) / TILE;

  // acc[db] (D x keys) += Y^T X: Y a staged [rows][D]^T LDS tile (rows d, queries in C-layout
  // order), X a C-layout (queries x keys) tile. With split, X also enters as its rounding residual.
  auto acc_t = [&](f32x16 (&acc)[DB], const elem* yt, const f32x16& x, bool split) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s) acc[db] = OP::mma(OP::ld_perm(yt, LDV, db * 32 + n, h, s), OP::from_acc(x, s), acc[db]);
    if constexpr (OP::SPLIT) {
      if (split) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int s = 0; s < AS; ++s)
            acc[db] = OP::mma(OP::ld_perm(yt, LDV, db * 32 + n, h, s), OP::from_acc_lo(x, s), acc[db]);
      }
    }
  };

  // dz (C layout, queries x keys) -> LDS -> dQ tile += dz K -> atomics into dq rows of qb. With
  // split, the rounding residual of dz takes a second pass through LDS.
  auto dq_update = [&](const f32x16& dzv, const frag (&ktfr)[DB][AS], float* dqh, int qb, bool split) {
    f32x16 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = zero16();
#pragma unroll
    for (int i = 0; i < 16; ++i) zs[crow(i, h) * LDZ + n] = OP::to_elem(dzv[i]);
    lds_wave_sync();
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s) acc[db] = OP::mma(OP::ld_std(zs, LDZ, n, h, s), ktfr[db][s], acc[db]);
    if constexpr (OP::SPLIT) {
      if (split) {
        lds_wave_sync();
#pragma unroll
        for (int i = 0; i < 16; ++i) zs[crow(i, h) * LDZ + n] = OP::to_elem_lo(dzv[i]);
        lds_wave_sync();
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int s = 0; s < AS; ++s) acc[db] = OP::mma(OP::ld_std(zs, LDZ, n, h, s), ktfr[db][s], acc[db]);
      }
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = qb * TILE + crow(i, h);
        if (r < T) atomicAdd(dqh + (int64_t)r * D + db * 32 + n, acc[db][i]);
      }
    lds_wave_sync();
  };

  // Keys below `exempt` are never selected, so they gather attention from every later query and
  // their dV / dK sums run over all of them: their products take the split operands.
  const bool split_keys = key0 < exempt;

  for (int qb = NB - 1; qb >= qb_lo; --qb) {
    const int qbase = qb * TILE;
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t row = seq_row + hd0 + g;
      stage_rows<elem, D, LDK>(sQ[g], q + row * T * D, D, qbase, T, tid);
      stage_cols<elem, D, LDV>(sQt[g], qt + row * D * ldt, ldt, qbase, T, tid);
      stage_rows<elem, D, LDK>(sdO[g], dout + row * T * D, D, qbase, T, tid);
      stage_cols<elem, D, LDV>(sdOt[g], dot + row * D * ldt, ldt, qbase, T, tid);
      if (tid < TILE) {
        const int r = qbase + tid;
        sLse[g][tid] = (r < T) ? lse[row * T + r] : 0.f;
        sDb[g][tid] = (r < T) ? dbar[row * T + r] : 0.f;
      }
    }
    if (!has_h0) {
      stage_rows<elem, D, LDK>(sQ[G], q + seq_row * T * D, D, qbase, T, tid);
      stage_cols<elem, D, LDV>(sQt[G], qt + seq_row * D * ldt, ldt, qbase, T, tid);
    }
    __syncthreads();
    if (qbase + TILE - 1 < key0) continue;   // every query of the tile precedes every key
    const bool diag = (qbase < key0 + TILE - 1) || (qbase + TILE > T) || (key0 + TILE > T);

    // head 0 logits (queries x keys), selection gate and F (log2 units)
    const elem* q0s = has_h0 ? sQ[0] : sQ[G];
    f32x16 l0 = zero16();
#pragma unroll
    for (int s = 0; s < NS; ++s) l0 = OP::mma(OP::ld_std(q0s, LDK, n, h, s), has_h0 ? kf[0][s] : k0f[s], l0);
    f32x16 sel, fs;
    uint32_t gmask = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = qbase + crow(i, h);
      const float sv = l0[i] * scale;
      const bool gate = (r < T) && (j >= exempt) && (j < r) && (sv > 0.f);
      sel[i] = gate ? sv : 0.f;
      gmask |= gate ? (1u << i) : 0u;
    }
    {
      float gs[4], pg[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) gs[a] = ((sel[4 * a] + sel[4 * a + 1]) + sel[4 * a + 2]) + sel[4 * a + 3];
#pragma unroll
      for (int a = 0; a < 4; ++a) pg[a] = xor32(gs[a]);
      float run = (j < T) ? carry[((int64_t)b * NB + qb) * T + j] : 0.f;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float g_lo = h == 0 ? gs[a] : pg[a];   // rows 8a..8a+3
        const float g_hi = h == 0 ? pg[a] : gs[a];   // rows 8a+4..8a+7
        float p = (h == 0) ? run : run + g_lo;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          fs[4 * a + t] = p * LOG2E;
          p += sel[4 * a + t];
        }
        run = (run + g_lo) + g_hi;
      }
    }

    f32x16 dzsum = zero16();
    f32x16 dz0 = zero16();
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      const int g = has_h0 ? (gg + 1) % G : gg;   // head 0 last: its dK, dQ wait for g
      const int64_t row = seq_row + hd0 + g;
      f32x16 lg;
      if (has_h0 && g == 0) {
        lg = l0;
      } else {
        lg = zero16();
#pragma unroll
        for (int s = 0; s < NS; ++s) lg = OP::mma(OP::ld_std(sQ[g], LDK, n, h, s), kf[g][s], lg);
      }
      f32x16 dp = zero16();
#pragma unroll
      for (int s = 0; s < NS; ++s) dp = OP::mma(OP::ld_std(sdO[g], LDK, n, h, s), vf[g][s], dp);
      f32x16 pr, dz;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float4 ls = *reinterpret_cast<const float4*>(&sLse[g][8 * a + 4 * h]);
        const float4 dbv = *reinterpret_cast<const float4*>(&sDb[g][8 * a + 4 * h]);
        const float lsv[4] = {ls.x, ls.y, ls.z, ls.w};
        const float dbs[4] = {dbv.x, dbv.y, dbv.z, dbv.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int i = 4 * a + t;
          float p = fast_exp2(lg[i] * sl2 - fs[i] - lsv[t]);
          if (diag) {
            const int r = qbase + crow(i, h);
            if (j > r || r >= T || j >= T) p = 0.f;
          }
          pr[i] = p;
          dz[i] = p * (dp[i] - dbs[t]);
        }
      }
      // dV^T += dO^T P
      acc_t(dvt[g], sdOt[g], pr, split_keys);
#pragma unroll
      for (int i = 0; i < 16; ++i) dzsum[i] += dz[i];
      if (has_h0 && g == 0) {
        dz0 = dz;
      } else {
        acc_t(dkt[g], sQt[g], dz, split_keys);
        dq_update(dz, ktf[g], dq + row * T * D, qb, false);
      }
    }

    // U = ucarry + sum over later queries of the tile (reverse exclusive), g = -gate U
    f32x16 gpath;
    {
      float gs[4], pg[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) gs[a] = ((dzsum[4 * a + 3] + dzsum[4 * a + 2]) + dzsum[4 * a + 1]) + dzsum[4 * a];
#pragma unroll
      for (int a = 0; a < 4; ++a) pg[a] = xor32(gs[a]);
      float run = ucarry;
#pragma unroll
      for (int a = 3; a >= 0; --a) {
        const float g_lo = h == 0 ? gs[a] : pg[a];
        const float g_hi = h == 0 ? pg[a] : gs[a];
        float p = (h == 1) ? run : run + g_hi;
#pragma unroll
        for (int t = 3; t >= 0; --t) {
          const int i = 4 * a + t;
          gpath[i] = ((gmask >> i) & 1u) ? -p : 0.f;
          p += dzsum[i];
        }
        run = (run + g_hi) + g_lo;
      }
      ucarry = run;
    }

    // g sums dz over every later query of every head: it outgrows the dz tiles, so head 0's
    // products take it split (the group holding head 0 always, the others when some |g| > 1/4).
    if (has_h0) {
      f32x16 dzh;
#pragma unroll
      for (int i = 0; i < 16; ++i) dzh[i] = dz0[i] + gpath[i];
      acc_t(dkt[0], sQt[0], dzh, true);
      dq_update(dzh, ktf[0], dq + seq_row * T * D, qb, true);
    } else {
      bool big = false;
#pragma unroll
      for (int i = 0; i < 16; ++i) big |= fabsf(gpath[i]) > 0.25f;
      const bool split_g = __any(big);
      acc_t(dk0t, sQt[G], gpath, split_g);
      dq_update(gpath, k0tf, dq + seq_row * T * D, qb, split_g);
    }
  }

  if (j >= T) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t row = seq_row + hd0 + g;
    float* dkr = dk + (row * T + j) * D;
    float* dvr = dv + (row * T + j) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = db * 32 + 8 * a + 4 * h;
        *reinterpret_cast<float4*>(dkr + d) =
            make_float4(dkt[g][db][4 * a] * scale, dkt[g][db][4 * a + 1] * scale,
                        dkt[g][db][4 * a + 2] * scale, dkt[g][db][4 * a + 3] * scale);
        *reinterpret_cast<float4*>(dvr + d) =
            make_float4(dvt[g][db][4 * a], dvt[g][db][4 * a + 1], dvt[g][db][4 * a + 2], dvt[g][db][4 * a + 3]);
      }
  }
  if (!has_h0) {
    float* dst = dk0x + ((int64_t)b * T + j) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) atomicAdd(dst + db * 32 + crow(i, h), dk0t[db][i] * scale);
  }
}

// Gradients to the output dtype (bf16 or fp32): dq*scale, dk (+ head 0's share from other groups), dv.
__device__ __forceinline__ void store_grad(uint16_t* p, float x) { *p = OpBF16::to_elem(x); }
__device__ __forceinline__ void store_grad(float* p, float x) { *p = x; }

template <typename OUT>
__global__ __launch_bounds__(NTHREADS) void bwd_finish_kernel(
    const float* __restrict__ dq32, const float* __restrict__ dk32, const float* __restrict__ dv32,
    const float* __restrict__ dk0x, OUT* __restrict__ dq, OUT* __restrict__ dk, OUT* __restrict__ dv, int H,
    int64_t TD, int64_t total, float scale) {
  for (int64_t e = (int64_t)blockIdx.x * NTHREADS + threadIdx.x; e < total; e += (int64_t)gridDim.x * NTHREADS) {
    const int64_t row = e / TD;          // b*H + head
    const int64_t off = e - row * TD;
    float kv = dk32[e];
    if (row % H == 0) kv += dk0x[(row / H) * TD + off];
    store_grad(dq + e, dq32[e] * scale);
    store_grad(dk + e, kv);
    store_grad(dv + e, dv32[e]);
  }
}

// ---------------------------------------------------------------------------------------------
// Host side.

// Event timing of the main kernels, for measurement tools (sa_timing_enable / sa_timing_read).
// Off by default; when on, each timed launch is bracketed by a pair of HIP events recorded on the
// launch's own stream. The registry is the only mutable host state of the library.
struct TimingRegistry {
  std::mutex mu;
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events[SA_KERNEL_COUNT];
};
TimingRegistry& timing() {
  static TimingRegistry r;
  return r;
}

// Brackets one launch: construct before it, destroy after it (both on stream st).
class TimedLaunch {
 public:
  TimedLaunch(int kernel, hipStream_t st) : kernel_(kernel), st_(st) {
    TimingRegistry& r = timing();
    std::lock_guard<std::mutex> lock(r.mu);
    if (!r.on) return;
    if (hipEventCreate(&start_) != hipSuccess) return;
    if (hipEventCreate(&stop_) != hipSuccess) {
      (void)hipEventDestroy(start_);
      return;
    }
    active_ = hipEventRecord(start_, st_) == hipSuccess;
  }
  ~TimedLaunch() {
    if (!active_) return;
    TimingRegistry& r = timing();
    std::lock_guard<std::mutex> lock(r.mu);
    if (hipEventRecord(stop_, st_) == hipSuccess) r.events[kernel_].emplace_back(start_, stop_);
  }

 private:
  int kernel_;
  hipStream_t st_;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
  bool active_ = false;
};

inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int launch_status() { return hipGetLastError() == hipSuccess ? SA_OK : SA_ERR_LAUNCH; }

int auto_group(int dtype, int64_t D, int64_t heads, int requested, bool backward) {
  int g = requested;
  if (g <= 0) {
    if (dtype == SA_DTYPE_F32) g = 1;
    else if (backward) g = (D <= 32) ? 2 : 1;
    else g = (D <= 32) ? 4 : (D <= 64 ? 2 : 1);
  }
  int cap = (dtype == SA_DTYPE_F32) ? 1 : (backward ? 2 : 4);
  if (D >= 128 || (backward && D >= 64)) cap = 1;
  g = g > cap ? cap : g;
  while (g > 1 && (heads % g != 0)) g >>= 1;
  return g < 1 ? 1 : g;
}

template <class OP, int D>
int run_selection(const typename OP::elem* q, const typename OP::elem* k, float* carry, const float* state_in,
                  float* state_out, int64_t state_ld, int nseq, int H, int Tq, int Tk, int q_off, int exempt,
                  float scale, hipStream_t st) {
  const int NBq = (int)cdiv(Tq, TILE), NKT = (int)cdiv(Tk, TILE);
  const int RB = 8;
  dim3 g1((unsigned)cdiv(NKT, NWAVES), (unsigned)cdiv(NBq, RB), (unsigned)nseq);
  TimedLaunch timed(SA_KERNEL_SELECTION, st);
  hipLaunchKernelGGL((sel_colsum_kernel<OP, D>), g1, dim3(NTHREADS), 0, st, q, k, carry, H, Tq, Tk, q_off, exempt,
                     scale, RB);
  dim3 g2((unsigned)cdiv(Tk, NTHREADS), (unsigned)nseq);
  hipLaunchKernelGGL(sel_scan_kernel, g2, dim3(NTHREADS), 0, st, carry, state_in, state_out, state_ld, NBq, Tk,
                     q_off);
  return launch_status();
}

template <class OP, int D, int G>
void launch_fwd(const typename OP::elem* q, const typename OP::elem* k, const typename OP::elem* vt,
                const float* carry, float* out, float* rmax, float* rden, int nseq, int H, int Tq, int Tk,
                int q_off, int64_t ldv, int exempt, float scale, int damp_mode, float train_len, hipStream_t st) {
  const int NBq = (int)cdiv(Tq, TILE);
  dim3 grid((unsigned)cdiv(NBq, NWAVES), (unsigned)(nseq * (H / G)));
  TimedLaunch timed(SA_KERNEL_FORWARD, st);
  hipLaunchKernelGGL((fwd_kernel<OP, D, G>), grid, dim3(NTHREADS), 0, st, q, k, vt, carry, out, rmax, rden, H, Tq,
                     Tk, q_off, ldv, exempt, scale, damp_mode, train_len);
}

template <class OP, int D>
int forward_impl(const void* q_, const void* k_, const void* v_, float* out, float* rmax, float* rden,
                 float* carry, const float* state_in, float* state_out, int64_t state_ld, void* ws, int nseq,
                 int H, int Tq, int Tk, int q_off, float scale, int exempt, int group, int damp_mode,
                 float train_len, hipStream_t st) {
  using elem = typename OP::elem;
  const elem* q = static_cast<const elem*>(q_);
  const elem* k = static_cast<const elem*>(k_);
  const elem* v = static_cast<const elem*>(v_);
  const int64_t ldv = sa_transposed_ld(Tk);
  elem* vt = static_cast<elem*>(ws);
  dim3 gt((unsigned)cdiv(ldv, 64), (unsigned)(nseq * H));
  hipLaunchKernelGGL((transpose_kernel<elem, D>), gt, dim3(NTHREADS), 0, st, v, vt, Tk, ldv);
  int rc = run_selection<OP, D>(q, k, carry, state_in, state_out, state_ld, nseq, H, Tq, Tk, q_off, exempt, scale, st);
  if (rc) return rc;
  const int dtype = sizeof(elem) == 2 ? SA_DTYPE_BF16 : SA_DTYPE_F32;
  const int G = auto_group(dtype, D, H, group, false);
  if (G == 4) {
    if constexpr (sizeof(elem) == 2 && D <= 64)
      launch_fwd<OP, D, 4>(q, k, vt, carry, out, rmax, rden, nseq, H, Tq, Tk, q_off, ldv, exempt, scale, damp_mode,
                           train_len, st);
  } else if (G == 2) {
    if constexpr (sizeof(elem) == 2 && D <= 64)
      launch_fwd<OP, D, 2>(q, k, vt, carry, out, rmax, rden, nseq, H, Tq, Tk, q_off, ldv, exempt, scale, damp_mode,
                           train_len, st);
  } else {
    launch_fwd<OP, D, 1>(q, k, vt, carry, out, rmax, rden, nseq, H, Tq, Tk, q_off, ldv, exempt, scale, damp_mode,
                         train_len, st);
  }
  return launch_status();
}

struct BwdLayout {
  int64_t qt, dot, lse, dbar, dq, dk, dv, dk0x, total;
};

BwdLayout bwd_layout(int64_t nseq, int64_t heads, int64_t t, int64_t D, int64_t esize) {
  const int64_t R = nseq * heads, ldt = sa_transposed_ld(t);
  BwdLayout L;
  int64_t off = 0;
  auto take = [&](int64_t bytes) { int64_t o = off; off = align_up(off + bytes, 256); return o; };
  L.qt = take(R * D * ldt * esize);
  L.dot = take(R * D * ldt * esize);
  L.lse = take(R * t * 4);
  L.dbar = take(R * t * 4);
  L.dq = take(R * t * D * 4);
  L.dk = take(R * t * D * 4);
  L.dv = take(R * t * D * 4);
  L.dk0x = take(nseq * t * D * 4);
  L.total = off;
  return L;
}

template <class OP, int D, int G>
void launch_bwd(const typename OP::elem* q, const typename OP::elem* k, const typename OP::elem* v,
                const typename OP::elem* qt, const typename OP::elem* dout, const typename OP::elem* dot,
                const float* lse, const float* dbar, const float* carry, float* dq, float* dk, float* dv,
                float* dk0x, int nseq, int H, int T, int64_t ldt, int exempt, float scale, hipStream_t st) {
  dim3 grid((unsigned)cdiv(T, NWAVES * TILE), (unsigned)(nseq * (H / G)));
  TimedLaunch timed(SA_KERNEL_BACKWARD, st);
  hipLaunchKernelGGL((bwd_kernel<OP, D, G>), grid, dim3(NTHREADS), 0, st, q, k, v, qt, dout, dot, lse, dbar, carry,
                     dq, dk, dv, dk0x, H, T, ldt, exempt, scale);
}

template <class OP, int D>
int backward_impl(const void* q_, const void* k_, const void* v_, const float* out, const void* dout_,
                  const float* rmax, const float* rden, const float* carry, void* dq_, void* dk_, void* dv_,
                  void* ws, int nseq, int H, int T, float scale, int exempt, int group, int grad_dtype,
                  hipStream_t st) {
  using elem = typename OP::elem;
  const elem* q = static_cast<const elem*>(q_);
  const elem* k = static_cast<const elem*>(k_);
  const elem* v = static_cast<const elem*>(v_);
  const elem* dout = static_cast<const elem*>(dout_);
  const int64_t R = (int64_t)nseq * H, ldt = sa_transposed_ld(T);
  const BwdLayout L = bwd_layout(nseq, H, T, D, sizeof(elem));
  char* base = static_cast<char*>(ws);
  elem* qt = reinterpret_cast<elem*>(base + L.qt);
  elem* dot = reinterpret_cast<elem*>(base + L.dot);
  float* lse = reinterpret_cast<float*>(base + L.lse);
  float* dbar = reinterpret_cast<float*>(base + L.dbar);
  float* dq32 = reinterpret_cast<float*>(base + L.dq);
  float* dk32 = reinterpret_cast<float*>(base + L.dk);
  float* dv32 = reinterpret_cast<float*>(base + L.dv);
  float* dk0x = reinterpret_cast<float*>(base + L.dk0x);

  dim3 gt((unsigned)cdiv(ldt, 64), (unsigned)R);
  hipLaunchKernelGGL((transpose_kernel<elem, D>), gt, dim3(NTHREADS), 0, st, q, qt, T, ldt);
  hipLaunchKernelGGL((transpose_kernel<elem, D>), gt, dim3(NTHREADS), 0, st, dout, dot, T, ldt);
  hipLaunchKernelGGL((bwd_rowstats_kernel<OP, D>), dim3((unsigned)cdiv(R * T, NTHREADS)), dim3(NTHREADS), 0, st,
                     dout, out, rmax, rden, lse, dbar, R * T);
  // dq32 and dk0x are atomic targets
  hipLaunchKernelGGL(fill_zero_kernel, dim3(1024), dim3(NTHREADS), 0, st, reinterpret_cast<float4*>(dq32),
                     (int64_t)(R * T * D / 4));
  hipLaunchKernelGGL(fill_zero_kernel, dim3(256), dim3(NTHREADS), 0, st, reinterpret_cast<float4*>(dk0x),
                     (int64_t)((int64_t)nseq * T * D / 4));
  const int dtype = sizeof(elem) == 2 ? SA_DTYPE_BF16 : SA_DTYPE_F32;
  const int G = auto_group(dtype, D, H, group, true);
  if (G == 2) {
    if constexpr (sizeof(elem) == 2 && D <= 32)
      launch_bwd<OP, D, 2>(q, k, v, qt, dout, dot, lse, dbar, carry, dq32, dk32, dv32, dk0x, nseq, H, T, ldt, exempt,
                           scale, st);
  } else {
    launch_bwd<OP, D, 1>(q, k, v, qt, dout, dot, lse, dbar, carry, dq32, dk32, dv32, dk0x, nseq, H, T, ldt, exempt,
                         scale, st);
  }
  const int64_t total = R * T * D;
  const dim3 fgrid((unsigned)std::min<int64_t>(cdiv(total, NTHREADS), 8192));
  if (grad_dtype == SA_DTYPE_F32)
    hipLaunchKernelGGL((bwd_finish_kernel<float>), fgrid, dim3(NTHREADS), 0, st, dq32, dk32, dv32, dk0x,
                       static_cast<float*>(dq_), static_cast<float*>(dk_), static_cast<float*>(dv_), H,
                       (int64_t)T * D, total, scale);
  else
    hipLaunchKernelGGL((bwd_finish_kernel<uint16_t>), fgrid, dim3(NTHREADS), 0, st, dq32, dk32, dv32, dk0x,
                       static_cast<uint16_t*>(dq_), static_cast<uint16_t*>(dk_), static_cast<uint16_t*>(dv_), H,
                       (int64_t)T * D, total, scale);
  return launch_status();
}

bool valid_dims(int64_t nseq, int64_t heads, int64_t t) {
  const int64_t lim = (int64_t)1 << 30;
  return nseq >= 1 && heads >= 1 && t >= 1 && nseq < 65536 && heads < 65536 && t < lim && nseq * heads < 65536;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// C ABI

extern "C" {

int sa_abi_version(void) { return 2; }

int sa_timing_enable(int on) {
  TimingRegistry& r = timing();
  std::lock_guard<std::mutex> lock(r.mu);
  for (auto& list : r.events) {
    for (auto& ev : list) {
      (void)hipEventDestroy(ev.first);
      (void)hipEventDestroy(ev.second);
    }
    list.clear();
  }
  r.on = on != 0;
  return SA_OK;
}

int sa_timing_read(int kernel, double* total_ms, int64_t* launches) {
  if (kernel < 0 || kernel >= SA_KERNEL_COUNT || !total_ms || !launches) return SA_ERR_ARGUMENT;
  TimingRegistry& r = timing();
  std::lock_guard<std::mutex> lock(r.mu);
  double sum = 0.0;
  for (auto& ev : r.events[kernel]) {
    float ms = 0.f;
    if (hipEventSynchronize(ev.second) != hipSuccess || hipEventElapsedTime(&ms, ev.first, ev.second) != hipSuccess)
      return SA_ERR_LAUNCH;
    sum += ms;
  }
  *total_ms = sum;
  *launches = (int64_t)r.events[kernel].size();
  return SA_OK;
}

const char* sa_status_string(int status) {
  switch (status) {
    case SA_OK: return "ok";
    case SA_ERR_ARGUMENT: return "invalid argument (size, pointer or option)";
    case SA_ERR_HEAD_DIM: return "head_dim must be 32, 64 or 128 at the C ABI";
    case SA_ERR_DTYPE: return "unknown dtype code";
    case SA_ERR_WORKSPACE: return "workspace too small";
    case SA_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown status";
  }
}

int64_t sa_transposed_ld(int64_t t) { return align_up(t < 1 ? 1 : t, 64); }

int64_t sa_forward_workspace_bytes(int64_t nseq, int64_t heads, int64_t tk, int64_t head_dim, int dtype) {
  const int64_t es = dtype == SA_DTYPE_BF16 ? 2 : 4;
  return align_up(nseq * heads * head_dim * sa_transposed_ld(tk) * es, 256);
}

int sa_forward(const void* q, const void* k, const void* v, float* out, float* rmax, float* rden, float* carry,
               const float* state_in, float* state_out, int64_t state_ld, void* workspace,
               int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t tq, int64_t tk, int64_t q_offset,
               int64_t head_dim, float scale, int dtype, int exempt, int group, int damp_mode, int64_t train_len,
               void* stream) {
  if (!valid_dims(nseq, heads, tk) || tq < 1 || q_offset < 0 || q_offset + tq != tk) return SA_ERR_ARGUMENT;
  if (!q || !k || !v || !out || !rmax || !rden || !carry || !state_out || !workspace) return SA_ERR_ARGUMENT;
  if (q_offset > 0 && !state_in) return SA_ERR_ARGUMENT;
  if (state_ld < tk || exempt < 1 || damp_mode < 0 || damp_mode > 2 || (damp_mode && train_len < 1))
    return SA_ERR_ARGUMENT;
  if (!(scale > 0.f) || !(scale < INFINITY)) return SA_ERR_ARGUMENT;
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return SA_ERR_HEAD_DIM;
  if (workspace_bytes < sa_forward_workspace_bytes(nseq, heads, tk, head_dim, dtype)) return SA_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int ns = (int)nseq, H = (int)heads, Tq = (int)tq, Tk = (int)tk, qo = (int)q_offset;
  const float tl = (float)train_len;
#define SA_FWD(OPT, DD)                                                                                             \
  return forward_impl<OPT, DD>(q, k, v, out, rmax, rden, carry, state_in, state_out, state_ld, workspace, ns, H, Tq, \
                               Tk, qo, scale, exempt, group, damp_mode, tl, st)
  if (dtype == SA_DTYPE_BF16) {
    if (head_dim == 32) SA_FWD(OpBF16, 32);
    if (head_dim == 64) SA_FWD(OpBF16, 64);
    SA_FWD(OpBF16, 128);
  } else {
    if (head_dim == 32) SA_FWD(OpF32, 32);
    if (head_dim == 64) SA_FWD(OpF32, 64);
    SA_FWD(OpF32, 128);
  }
#undef SA_FWD
}

int64_t sa_backward_workspace_bytes(int64_t nseq, int64_t heads, int64_t t, int64_t head_dim, int dtype) {
  return bwd_layout(nseq, heads, t, head_dim, dtype == SA_DTYPE_BF16 ? 2 : 4).total;
}

int sa_backward(const void* q, const void* k, const void* v, const float* out, const void* dout, const float* rmax,
                const float* rden, const float* carry, void* dq, void* dk, void* dv, void* workspace,
                int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t t, int64_t head_dim, float scale,
                int dtype, int grad_dtype, int exempt, int group, void* stream) {
  if (!valid_dims(nseq, heads, t) || exempt < 1) return SA_ERR_ARGUMENT;
  if (!(scale > 0.f) || !(scale < INFINITY)) return SA_ERR_ARGUMENT;
  if (!q || !k || !v || !out || !dout || !rmax || !rden || !carry || !dq || !dk || !dv || !workspace)
    return SA_ERR_ARGUMENT;
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (grad_dtype != SA_DTYPE_BF16 && grad_dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return SA_ERR_HEAD_DIM;
  if (workspace_bytes < sa_backward_workspace_bytes(nseq, heads, t, head_dim, dtype)) return SA_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int ns = (int)nseq, H = (int)heads, T = (int)t;
#define SA_BWD(OPT, DD) \
  return backward_impl<OPT, DD>(q, k, v, out, dout, rmax, rden, carry, dq, dk, dv, workspace, ns, H, T, scale, exempt, \
                                group, grad_dtype, st)
  if (dtype == SA_DTYPE_BF16) {
    if (head_dim == 32) SA_BWD(OpBF16, 32);
    if (head_dim == 64) SA_BWD(OpBF16, 64);
    SA_BWD(OpBF16, 128);
  } else {
    if (head_dim == 32) SA_BWD(OpF32, 32);
    if (head_dim == 64) SA_BWD(OpF32, 64);
    SA_BWD(OpF32, 128);
  }
#undef SA_BWD
}

}  // extern "C"

// Selective Attention for MI355X (gfx950): selection scan, forward, chunked prefill, backward.
//
// Operator (reference src/selective_attention/kernels.py:61-83, docs/kernel.md:32-46):
//   L_h = s Q_h K_h^T (causal),  S = relu(L_0) on E <= j < r,  F[i,j] = sum_{r<i} S[r,j],
//   O_h = softmax(L_h - F) V_h.
//
// Kernels (all 256 threads = 4 wavefronts of 64; MFMA 32x32 tiles; the attention kernels order
// their workgroups so that each XCD's L2 serves a contiguous range of heads):
//   sel_colsum   head 0, one 32x32 (queries x keys) tile per step: column sums of S per
//                32-query block -> colsum[b][rb][j]
//   sel_scan     exclusive running sum of colsum over query blocks, seeded by the carried
//                per-key state -> carry[b][rb][j], state_out[b][j]
//   fwd          query-parallel. A wavefront owns 32 queries of G heads. Logit tiles are
//                built transposed (keys x queries) so each lane holds one query: the online
//                softmax row statistics stay in-lane, and O^T = V^T P^T takes P straight from
//                the accumulator registers. Head 0's logits are built (queries x keys) instead,
//                so the selection's prefix over queries runs down each lane's registers; F then
//                reaches the softmax layout through the wavefront's LDS rows.
//   bwd_kv       key-parallel. A wavefront owns 32 keys of G heads and sweeps the query tiles
//                last to first. Tiles are (queries x keys), so the selection prefix F and the
//                suffix U = sum_h sum_{i>r} dz_h[i,j] run down registers. dK, dV (and the
//                group's share of head 0's dK) stay in registers; K, V rows sit in LDS. U is
//                checkpointed per query tile for bwd_dq.
//   bwd_dq       query-parallel. A wavefront owns 32 queries and walks the key tiles up to its
//                diagonal, recomputing P, dz and the selection gradient g from the key side's
//                U checkpoints; dQ = dz K takes dz through a per-wavefront LDS tile.
//   bwd_finish   gradient epilogue: scale, add head 0's shares, convert to the output dtype.
// The group holding head 0 folds g = -gate*U into head 0's own dz; every other group stores its
// share of head 0's gradients in a slot of its own, and bwd_finish sums the slots in a fixed order
// (no atomics: the backward is bitwise repeatable).
//
// MFMA operand layouts used throughout (v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x2_f32):
//   C (32x32, 16 fp32 per lane): lane l holds column l%32, rows crow(i, l/32), i = 0..15,
//                                crow(i,h) = 8*(i/4) + 4*h + i%4.
//   A (32xK) / B (Kx32):         lane l holds row (A) / column (B) l%32 and K elements
//                                [KS*step + (KS/2)*h, +KS/2) with KS = 16 (bf16) or 2 (fp32).
// A C-layout tile fed back as a B operand keeps its registers in place; the matching A operand
// is then read with the C layout's row order (ld_perm; bf16 tiles read that way are staged with
// their columns in that order, ColTile::store_crow, so a fragment is one 16-byte read).


#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "sa_host.h"

namespace {

using namespace sa_host;

typedef __bf16 bf16_t;
typedef bf16_t bf16x8 __attribute__((__vector_size__(8 * sizeof(bf16_t))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ int crow(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

// The values of lanes 0-31 (lo) and of lanes 32-63 (hi) of the same column, in every lane
// (one v_permlane32_swap).
struct Halves {
  float lo, hi;
};
__device__ __forceinline__ Halves halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return {__int_as_float(r[0]), __int_as_float(r[1])};
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Word 3 of a raw buffer resource on gfx950 (32-bit data format; offsets in bytes, range-checked
// against the resource's byte count: loads past it return zero).
constexpr int RSRC_WORD3 = 0x00020000;

// A 32 x 32 bf16 tile kept transposed in LDS for the transposing read ds_read_b64_tr_b16: rows of
// 32 elements (64 bytes), the 8-byte chunk c of row r stored at chunk c ^ sw(r / 2 mod 8), sw(a) =
// 4 (a mod 2) + a / 2. The read gives lane i of each 16-lane group, element t, the element i % 4
// of the 8 bytes that lane 4t + i/4 of the group addresses (measured on gfx950). The 8-byte
// lane-per-row writes go to the banks 16 lanes at a time (32 banks of 4 bytes, as measured with the
// bank-conflict counter): sixteen consecutive rows then hold one chunk in 16 distinct bank pairs
// (rows of one parity take distinct chunks); a transposing read of four consecutive rows, chunks
// 0-3 or 4-7, finds the two rows of each parity on opposite halves of the row.
__device__ __forceinline__ int trt_off(int r, int c) {
  const int a = (r >> 1) & 7;
  return r * 32 + ((c ^ (((a & 1) << 2) | (a >> 1))) << 2);
}

typedef short short4v __attribute__((ext_vector_type(4)));

// Writes a C-layout tile x (lane = column n, element i = row crow(i, h)) transposed: row n of the
// LDS tile holds column n of x, 4 consecutive rows of x per 8-byte write. LO: the rounding
// residuals x - bf16(x) instead.
template <bool LO>
__device__ __forceinline__ void put_tr(uint16_t* t, const f32x16& x, int n, int h) {
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    typedef bf16_t bf16x4 __attribute__((__vector_size__(4 * sizeof(bf16_t))));
    bf16x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float f = x[4 * a + e];
      v[e] = LO ? (bf16_t)(f - (float)(bf16_t)f) : (bf16_t)f;
    }
    *reinterpret_cast<bf16x4*>(t + trt_off(n, 2 * a + h)) = v;
  }
}

// The A (or B) operand of K step s read from such a tile: lane l gets row l % 32 of the
// untransposed tile, elements 16s + 8(l / 32) + 0..7, in order.
__device__ __forceinline__ bf16x8 get_tr(const uint16_t* t, int lane, int s) {
  const int g = lane >> 4, k = lane & 15;
  const int n0 = 16 * (g & 1), hh = g >> 1;
  bf16x8 f;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = 16 * s + 8 * hh + 4 * hf + (k >> 2);
    typedef __attribute__((address_space(3))) short4v* lds_s4;
    const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(t + trt_off(r, (n0 >> 2) + (k & 3))));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const short x = v[e];
      f[4 * hf + e] = *reinterpret_cast<const bf16_t*>(&x);
    }
  }
  return f;
}

// Element i = s[crow(i, h)]: a C-layout tile whose rows take the values of a 32-entry LDS row
// vector (four 16-byte reads).
__device__ __forceinline__ f32x16 rows16(const float* s, int h) {
  f32x16 r;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const float4 v = *reinterpret_cast<const float4*>(s + 8 * a + 4 * h);
    r[4 * a] = v.x;
    r[4 * a + 1] = v.y;
    r[4 * a + 2] = v.z;
    r[4 * a + 3] = v.w;
  }
  return r;
}

// The wavefront index within the workgroup, as a value the compiler knows is uniform across the
// wavefront (threadIdx.x / 64 is, but divergence analysis cannot see it): tile flags derived from
// it become scalar branches instead of per-lane exec masks.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Wavefront-local ordering of LDS traffic (writes by some lanes, reads by others).
__device__ __forceinline__ void lds_wave_sync() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}
// The same ordering without the wait: the LDS performs one wavefront's operations in issue order,
// so a read issued after a write of the same wavefront sees it, and a later write cannot overtake an
// earlier read; only the compiler must keep the accesses in program order. (The wait drained every
// outstanding LDS read of the wavefront, operand reads of the next product included: measured, the
// query-side backward at C2 runs 1.4% faster without it, all GPU tests unchanged.)
__device__ __forceinline__ void lds_wave_order() { __asm__ volatile("" ::: "memory"); }

// ---------------------------------------------------------------------------------------------
// Operand traits: bf16 storage -> bf16 MFMA; fp32 storage -> fp32 MFMA.

struct OpBF16 {
  typedef uint16_t elem;
  typedef bf16x8 frag;
  static constexpr int KS = 16;
  static constexpr int KPAD = 8;     // LDS row padding (elements) of [rows][D] tiles
  static constexpr int TPAD = 8;     // LDS row padding (elements) of [rows][32] tiles: 80-byte rows,
                                     // 16-byte aligned, distinct banks for 16 rows

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
  // Row r, K elements in C-layout row order for step s -- columns [16s+4h, +4) and [16s+8+4h, +4)
  // -- from a tile whose columns were stored in that order (ColTile::store_crow): one 16-byte read.
  static __device__ __forceinline__ frag ld_perm(const elem* p, int64_t ld, int r, int h, int s) {
    return *reinterpret_cast<const frag*>(p + r * ld + s * 16 + 8 * h);
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
    return p[r * ld + crow(s, h)];   // a standard-order tile (ColTile::store_crow stores fp32 as is)
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

// The dispatcher deals workgroups round-robin to the 8 XCDs, each with its own L2. The selection
// kernels and the generic forward remap the linear workgroup id so that every XCD takes a contiguous
// range of the (head group, block) order instead: the workgroups one L2 serves at a time then belong
// to one or two heads and share that head's tiles (the direct-load forward's order is part_block, the
// backward kernels' work_order_block, below).
constexpr int NXCD = 8;
struct BlockXY {
  int x, y;
};
__device__ __forceinline__ BlockXY xcd_block() {
  const int gx = gridDim.x, n = gx * gridDim.y;
  const int l = blockIdx.x + gx * blockIdx.y;
  const int per = n / NXCD;
  const int m = (l < per * NXCD) ? (l % NXCD) * per + l / NXCD : l;
  return {m % gx, m / gx};
}

// The backward kernels' order: x-major (x the block, whose work falls as x grows; y the head row),
// so the round-robin deal gives every XCD every eighth workgroup of a list sorted by work: each XCD
// runs its share longest first and the XCDs' shares stay even whatever the head count. (With the
// contiguous ranges of xcd_block, 12 heads leave one XCD a third more work than the mean: the
// backward at the reference's 12-head geometry ran as long as at 16 heads.) An XCD still serves
// few heads at a time -- heads i and i + 8 at a multiple of 8 -- whose tiles it shares in its L2.
__device__ __forceinline__ BlockXY work_order_block() {
  const int gy = gridDim.y;
  const int l = blockIdx.x + gridDim.x * blockIdx.y;
  return {l / gy, l % gy};
}

// work_order_block with each XCD's share (every eighth workgroup of the longest-first list, n of
// them) dispatched in a different order when `slots` (the workgroups an XCD runs at once) is
// nonzero: its `slots` longest first, as before, then the shortest third of the rest, shortest
// first, then the middle third, longest first. The dispatcher hands an XCD's next workgroup to
// whichever slot frees first, so with about three workgroups per slot (the 12 heads of the
// reference's model at 16384 tokens) a slot that ran a short first workgroup collects a run of the
// shortest ones before the middle third arrives, and the slots end closer together than with the
// longest-first order, whose third round leaves the spread of the middle third (a list-scheduling
// simulation: 1.03x the balanced share against 1.11x). The query-side kernel takes it (one
// workgroup per CU; the host passes `slots` only in that regime, bwd_snake_slots): at d768 1.28 ->
// 1.18 ms per layer. The key side, two workgroups per CU, keeps the longest-first order: a
// workgroup left alone on its CU speeds up once its CU-mate finishes, which already evens its
// slots (1.20 ms there, three quarters of its 16-head time), and the other order ran it 3% slower.
__device__ __forceinline__ BlockXY work_order_block(int slots) {
  if (slots <= 0) return work_order_block();
  const int gy = gridDim.y, total = gridDim.x * gy;
  const int l = blockIdx.x + gridDim.x * blockIdx.y;
  const int x8 = l % NXCD, p = l / NXCD;             // this XCD's p-th dispatch
  const int n = (total - x8 + NXCD - 1) / NXCD;      // workgroups of this XCD
  int q = p;                                         // rank in the XCD's longest-first list
  if (p >= slots && n > slots) {
    const int rest = n - slots, n_low = rest - rest / 2, pp = p - slots;
    q = (pp < n_low) ? n - 1 - pp : slots + (pp - n_low);
  }
  const int g = q * NXCD + x8;
  return {g / gy, g % gy};
}

// The direct-load forward's order: every XCD takes an equal share of the work from as few head
// groups as that allows, longest first. Each row y (one head group of one sequence, its blocks x
// ordered longest first) is cut into P parts by x mod P, P = 8 / gcd(gy, 8), so that the gy * P
// parts divide evenly over the 8 XCDs; the parts of a row hold nearly equal work. XCD i takes parts
// [i m, i m + m), m = gy P / 8 (one row's worth or a little more), and runs them x-major: block by
// block, longest first. With 6 or 12 rows (the 12 heads of the reference's model, in pairs)
// xcd_block's contiguous ranges give one XCD the long blocks of a row and another its short ones
// (measured: a third more work on the busiest XCD). With gy a multiple of 8 (P = 1) every XCD takes
// whole rows and xcd_block's order, one row after another, is kept: interleaving an XCD's rows
// doubled the forward's HBM fetches at 32 rows (C5's). A grid whose x extent P does not divide falls
// back to xcd_block too.
__device__ __forceinline__ BlockXY part_block() {
  const int gx = gridDim.x, gy = gridDim.y;
  const int P = NXCD >> min(__builtin_ctz((unsigned)gy), 3);   // 8 / gcd(gy, 8)
  if (P == 1 || gx % P != 0) return xcd_block();
  const int m = gy * P / NXCD;
  const int l = blockIdx.x + gx * blockIdx.y;
  const int r = l / NXCD;
  const int part = (l % NXCD) * m + r % m;
  return {part % P + (r / m) * P, part / P};
}

// Unpadded LDS rows of 64 bf16 (eight 16-byte chunks), chunk c of row r stored at chunk position
// (c + r/2) mod 8. A 16-byte read serves 16 lanes per pass from 64 four-byte banks (256 bytes):
// two consecutive 128-byte rows already fall in different halves, and the rotation by r/2 puts the
// eight row pairs of a pass on distinct chunks, so a lane-per-row fragment read (every lane the
// same logical chunk) is conflict-free, as with a padded row stride, without the padding's bytes
// (measured: a rotation by r or an XOR by r mod 8 takes twice the cycles).
__device__ __forceinline__ int swz64(int r, int c) { return r * 64 + (((c + (r >> 1)) & 7) << 3); }

// Unpadded LDS rows of 64 bf16 read both ways: by lane-per-row fragment reads and by transposing
// reads (get_trq). Chunk c of row r is stored at chunk c ^ f(r), f(r) = 2 (r mod 4) ^ (r/4 mod 4).
// A 16-byte read of one chunk by 16 consecutive rows (16 lanes per pass over 64 four-byte banks):
// the eight rows of each parity take eight distinct chunks. A transposing read of four consecutive
// rows, an aligned 32-byte column range of each (16 lanes per pass over 32 banks, or 32 lanes over
// 64 banks reading 64 bytes of each row): f(r) / 2 takes four distinct values on the four rows, and
// rows two apart differ in bit 2 of f, so every pass touches distinct banks.
__device__ __forceinline__ int swzq(int r, int c) { return r * 64 + ((c ^ (((r & 3) << 1) ^ ((r >> 2) & 3))) << 3); }

typedef __attribute__((address_space(3))) void* lds_void_ptr;
// The LDS address of a pointer into a __shared__ variable, as the address-space-3 pointer the direct
// loads take: the low 32 bits of the generic address (a plain cast tests the pointer for null, a
// compare and select on the scalar unit per load).
__device__ __forceinline__ lds_void_ptr lds_ptr(const void* p) { return (lds_void_ptr)(uint32_t)(uintptr_t)p; }

// A buffer resource over `bytes` bytes from p (loads past them read zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, RSRC_WORD3);
}

// Direct loads into LDS: one instruction fills 64 consecutive 16-byte slots (1 KB) from the given
// LDS base, lane l slot l (measured lane layout on gfx950); each lane reads the global chunk that
// belongs in its slot, through a buffer resource (the scalar offset counts in the range check,
// measured: rows past the resource load zero). A [32][64] bf16 tile takes four such loads, parts
// m = 0..3.
//   rows64: a [32 rows][64] tile in swz64 layout from rows row0.. of a row-major matrix (row stride
//           ld elements). Slot 64m + l holds row 8m + l/8, stored chunk l mod 8, so logical chunk
//           (l mod 8 - l/16 - 4m) mod 8: c0 = (l mod 8 - l/16) mod 8 for even m, c0 ^ 4 for odd m.
// A wavefront always loads the same part m of every tile, so the lane's offset is chosen once, as a
// value (a per-load choice between two fields compiled into a choice of addresses, which kept the
// pair in scratch memory and made every load wait for a scratch read first).
struct RowsLane {
  int v;   // the lane's byte offset for part m
  __device__ __forceinline__ RowsLane(int ld, int lane, int m) {
    const int c0 = ((lane & 7) - (lane >> 4)) & 7;
    v = ((lane >> 3) * ld + 8 * ((m & 1) ? (c0 ^ 4) : c0)) * 2;
  }
};
__device__ __forceinline__ void g2l_rows64(uint16_t* tile, __amdgpu_buffer_rsrc_t rs, const RowsLane& rl, int ld,
                                           int row0, int m) {   // m: the part rl was made for
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds_ptr(tile + 512 * m), 16, rl.v, (row0 + 8 * m) * ld * 2, 0,
                                           0);
}
//   rowsq: a [32 rows][64] tile in swzq layout, as rows64. Slot 64m + l holds row r = 8m + l/8,
//          stored chunk l mod 8, so logical chunk (l mod 8) ^ f(r), f(r) = 2 (l/8 mod 4) ^ (l/32)
//          ^ 2 (m mod 2): c0 = (l mod 8) ^ 2 (l/8 mod 4) ^ l/32 for even m, c0 ^ 2 for odd m.
struct RowsLaneQ {
  int v;   // the lane's byte offset for part m (see RowsLane)
  __device__ __forceinline__ RowsLaneQ(int ld, int lane, int m) {
    const int c0 = (lane & 7) ^ (((lane >> 3) & 3) << 1) ^ (lane >> 5);
    v = ((lane >> 3) * ld + 8 * ((m & 1) ? (c0 ^ 2) : c0)) * 2;
  }
};
__device__ __forceinline__ void g2l_rowsq(uint16_t* tile, __amdgpu_buffer_rsrc_t rs, const RowsLaneQ& rl, int ld,
                                          int row0, int m) {   // m: the part rl was made for
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds_ptr(tile + 512 * m), 16, rl.v, (row0 + 8 * m) * ld * 2, 0,
                                           0);
}
// An operand of K step s of a product over the rows of a [32 rows][64] swzq tile Y (Y^T X, or X Y):
// lane l gets column 32 db + l % 32 of the tile, rows 16s + 8(l / 32) + 0..7 in order, or with
// CROW the rows a C-layout tile's fragment holds in the accumulator's row order (X entering from
// registers, OpBF16::from_acc): element e is row crow(8s + e, l / 32) = 16s + 8(e / 4) + 4(l / 32)
// + e % 4. Two transposing reads, four rows each: lane i of a 16-lane group gets, as element t,
// element i % 4 of the 8 bytes that lane 4t + i/4 of the group addresses, so lane k of the group
// addresses row base + k/4, columns 4 (k mod 4) .. +3 of the group's 16 (measured lane layout, see
// get_tr).
template <bool CROW>
__device__ __forceinline__ bf16x8 get_trq(const uint16_t* t, int lane, int db, int s) {
  const int g = lane >> 4, k = lane & 15;
  const int c = 4 * db + 2 * (g & 1) + ((k & 3) >> 1);   // the 16-byte chunk of the lane's 4 columns
  bf16x8 f;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = CROW ? 16 * s + 8 * hf + 4 * (g >> 1) + (k >> 2) : 16 * s + 8 * (g >> 1) + 4 * hf + (k >> 2);
    typedef __attribute__((address_space(3))) short4v* lds_s4;
    const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(t + swzq(r, c) + 4 * (k & 1)));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const short x = v[e];
      f[4 * hf + e] = *reinterpret_cast<const bf16_t*>(&x);
    }
  }
  return f;
}
// the wavefront's outstanding vector-memory operations (the direct loads included) have completed
__device__ __forceinline__ void wait_loads() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Register-staged tiles for software pipelining: load() issues a tile's global loads into registers
// (each thread owns PER 16-byte chunks), store() later writes them to LDS, so the loads of the next
// tile are in flight while the current one is computed.

// [32 rows][COLS] of a row-major global matrix (row stride gld); rows >= nrows read as zero: the
// loads go through a buffer resource over the nrows rows (nrows * gld elements below 2 GiB, checked
// by the host), so there is no bound check and the offsets are 32-bit (the lane's own part fixed,
// the tile's in a scalar register).
template <typename E, int COLS>
struct RowTile {
  static constexpr int EPC = 16 / sizeof(E);
  static constexpr int CPR = COLS / EPC;
  static constexpr int NCH = TILE * CPR;
  static constexpr int PER = (NCH + NTHREADS - 1) / NTHREADS;
  uint4 v[PER];
  __device__ __forceinline__ void load(const E* g, int64_t gld, int row0, int nrows, int tid) {
    const int ld = (int)gld;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)g, 0, nrows * ld * (int)sizeof(E), RSRC_WORD3);
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int c = (tid + p * NTHREADS) % NCH;   // PER * NTHREADS > NCH only for small tiles
      const int r = c / CPR, cc = (c % CPR) * EPC;
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(rs, (r * ld + cc) * (int)sizeof(E),
                                                           row0 * ld * (int)sizeof(E), 0);
      v[p] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  }
  template <int SLD>
  __device__ __forceinline__ void store(E* s, int tid) const {
    static_assert((SLD * sizeof(E)) % 16 == 0, "row stride must keep 16-byte alignment");
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int c = tid + p * NTHREADS;
      const int r = (c % NCH) / CPR, cc = (c % CPR) * EPC;
      if (NCH % NTHREADS == 0 || c < NCH) *reinterpret_cast<uint4*>(s + r * SLD + cc) = v[p];
    }
  }
};

// Columns col0..col0+31 of ROWS rows of one of this library's transposed copies: row stride gld,
// a multiple of 64 elements, zero-filled past the sequence, so every 16-byte chunk is in bounds and
// the load needs no check. Buffer loads as for RowTile: 32-bit offsets, the lane's part fixed.
template <typename E, int ROWS>
struct ColTile {
  static constexpr int EPC = 16 / sizeof(E);
  static constexpr int CPR = TILE / EPC;
  static constexpr int NCH = ROWS * CPR;
  static constexpr int PER = (NCH + NTHREADS - 1) / NTHREADS;
  uint4 v[PER];
  __device__ __forceinline__ void load(const E* g, int64_t gld, int col0, int tid) {
    const int ld = (int)gld;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)g, 0, ROWS * ld * (int)sizeof(E), RSRC_WORD3);
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int c = (tid + p * NTHREADS) % NCH;
      const int r = c / CPR, cc = (c % CPR) * EPC;
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(rs, (r * ld + cc) * (int)sizeof(E),
                                                           col0 * (int)sizeof(E), 0);
      v[p] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  }
  template <int SLD>
  __device__ __forceinline__ void store(E* s, int tid) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int c = tid + p * NTHREADS;
      const int r = (c % NCH) / CPR, cc = (c % CPR) * EPC;
      if (!(NCH % NTHREADS == 0 || c < NCH)) continue;
      E* dst = s + r * SLD + cc;
      if constexpr (sizeof(E) == 2) {
        static_assert((SLD * 2) % 8 == 0, "bf16 column tiles need 8-byte row alignment");
        reinterpret_cast<uint2*>(dst)[0] = make_uint2(v[p].x, v[p].y);
        reinterpret_cast<uint2*>(dst)[1] = make_uint2(v[p].z, v[p].w);
      } else {
        union { uint4 q; E e[EPC]; } u;
        u.q = v[p];
#pragma unroll
        for (int e = 0; e < EPC; ++e) dst[e] = u.e[e];
      }
    }
  }
  // bf16: the columns of each 16-column block in C-layout row order -- groups of four columns
  // 0, 2, 1, 3 -- so OpBF16::ld_perm reads a fragment with one 16-byte read; fp32 as store().
  template <int SLD>
  __device__ __forceinline__ void store_crow(E* s, int tid) const {
    if constexpr (sizeof(E) != 2) {
      store<SLD>(s, tid);
    } else {
      static_assert((SLD * 2) % 16 == 0, "C-layout-order tiles need 16-byte row alignment");
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int c = tid + p * NTHREADS;
        const int r = (c % NCH) / CPR, cc = (c % CPR) * EPC;
        if (!(NCH % NTHREADS == 0 || c < NCH)) continue;
        // cc is a multiple of 8: its groups of four are 2(cc%16)/8 and that + 1, at 0 -> 0, 1 -> 2,
        // 2 -> 1, 3 -> 3
        const int a0 = (cc & 15) >> 2;
        const int a1 = a0 + 1;
        E* row = s + r * SLD + (cc & ~15);
        reinterpret_cast<uint2*>(row + 4 * (((a0 & 1) << 1) | (a0 >> 1)))[0] = make_uint2(v[p].x, v[p].y);
        reinterpret_cast<uint2*>(row + 4 * (((a1 & 1) << 1) | (a1 >> 1)))[0] = make_uint2(v[p].z, v[p].w);
      }
    }
  }
};

// ---------------------------------------------------------------------------------------------
// Lane scans (DPP) across the 32 lanes of each half-wavefront.

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_shift(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}

// Exclusive prefix sums over lanes 0..31 and, separately, 32..63, of 16 values at once, step by step
// across the 16 (each DPP step then has 16 independent instructions and no read-after-write
// hazard waits between them).
__device__ __forceinline__ void excl_scan32x16(f32x16& x) {
  f32x16 s = x;
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] += dpp_shift<0x111, 0xF>(s[i]);   // row_shr:1
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] += dpp_shift<0x112, 0xF>(s[i]);   // row_shr:2
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] += dpp_shift<0x114, 0xF>(s[i]);   // row_shr:4
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] += dpp_shift<0x118, 0xF>(s[i]);   // row_shr:8
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] += dpp_shift<0x142, 0xA>(s[i]);   // row_bcast:15 into rows 1, 3
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = s[i] - x[i];
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
// One key block's selection summed over a query block: acc holds the raw logits (queries x keys, C
// layout, lane = key j; element i is the block's query crow(i, h)), relu'd in unscaled logit units
// (relu(s x) = s relu(x), s > 0); on tiles that are not interior, only the pairs with
// exempt <= j < query count: crow(i, 0) > thr, thr = j - (first query of the block) - 4h (32 when j
// is exempt). Queries past the end and keys past the end hold zero rows, so their logits add
// nothing. Summed in a fixed tree order, the wavefront's halves added, times the scale (the same
// value in both lanes of key j). The column-sum and one-pass carry kernels both take it, so their
// sums agree bit for bit.
__device__ __forceinline__ float block_selection_sum(const f32x16& acc, bool interior, int thr, float scale) {
  f32x16 s;
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = __builtin_amdgcn_fmed3f(acc[i], 0.f, 3.0e38f);
  if (!interior) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = crow(i, 0) > thr ? s[i] : 0.f;
  }
  float p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = s[2 * i] + s[2 * i + 1];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = p[2 * i] + p[2 * i + 1];
  const Halves cs = halves((p[0] + p[1]) + (p[2] + p[3]));
  return (cs.lo + cs.hi) * scale;
}

// ---------------------------------------------------------------------------------------------
// Selection column sums: colsum[b][rb][j] = sum over the queries r of block rb (chunk-relative)
// of S[r, j]. One wavefront per key block (its K rows in registers); a workgroup walks RB query
// blocks, each staged once in LDS for its four wavefronts while the next one loads.
constexpr int SEL_RB = 8;   // query blocks per workgroup

template <class OP, int D>
__global__ __launch_bounds__(NTHREADS) void sel_colsum_kernel(
    const typename OP::elem* __restrict__ q, const typename OP::elem* __restrict__ k,
    float* __restrict__ colsum, int H, int Tq, int Tk, Strides qs, Strides ks, int q_off, int exempt, float scale,
    int RB) {
  using elem = typename OP::elem;
  using frag = typename OP::frag;
  constexpr int NS = D / OP::KS;
  constexpr int LDK = D + OP::KPAD;
  __shared__ __attribute__((aligned(16))) elem sQ[2][TILE * LDK];   // query blocks, double-buffered
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int NKT = (Tk + TILE - 1) / TILE;
  const int NBq = (Tq + TILE - 1) / TILE;
  const int kb = blockIdx.x * NWAVES + wave;   // (a wavefront past the last key block only stages)
  const int b = blockIdx.z;
  const elem* q0 = q + qs.at(b, 0);
  const elem* k0 = k + ks.at(b, 0);
  const int j = kb * TILE + n;
  const int kbase = kb * TILE;

  frag kf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) kf[s] = ld_std_bounded<OP>(k0, ks.row, kbase + n, Tk, h, s);
  // a tile is interior when every pair passes: keys before every query, not exempt, queries
  // before the end (keys past the end hold zero rows, their sums are never written)
  const int rb0 = blockIdx.y * RB, rb_end = min(NBq, rb0 + RB);
  RowTile<elem, D> nQ;
  if (rb0 < rb_end) {
    nQ.load(q0, qs.row, rb0 * TILE, Tq, tid);
    nQ.template store<LDK>(sQ[0], tid);
  }
  __syncthreads();
  for (int rb = rb0; rb < rb_end; ++rb) {
    const int buf = (rb - rb0) & 1;
    // the next block, into registers, unconditionally (past the end it reads zero rows, unused): a
    // conditional load made the compiler wait for it at the join before this block's products
    nQ.load(q0, qs.row, (rb + 1) * TILE, Tq, tid);
    float cs = 0.f;
    const int qbase = q_off + rb * TILE;   // absolute position of the block's first query
    // the tile holds a selectable pair only if some query is after the first key
    if (kb < NKT && qbase + TILE - 1 > kbase) {
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < NS; ++s) acc = OP::mma(OP::ld_std(sQ[buf], LDK, n, h, s), kf[s], acc);
      const bool interior = qbase > kbase + TILE - 1 && kbase >= exempt;
      cs = block_selection_sum(acc, interior, j >= exempt ? j - qbase - 4 * h : 32, scale);
    }
    if (kb < NKT && h == 0 && j < Tk) colsum[((int64_t)b * NBq + rb) * Tk + j] = cs;
    if (rb + 1 < rb_end) nQ.template store<LDK>(sQ[buf ^ 1], tid);
    __syncthreads();
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
  constexpr int U = 16;   // blocks per step: their loads are issued together
  int rb = 0;
  for (; rb + U <= NBq; rb += U) {
    float c[U];
#pragma unroll
    for (int u = 0; u < U; ++u) c[u] = col[(int64_t)(rb + u) * Tk];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      col[(int64_t)(rb + u) * Tk] = run;
      run += c[u];
    }
  }
  for (; rb < NBq; ++rb) {
    const float c = col[(int64_t)rb * Tk];
    col[(int64_t)rb * Tk] = run;
    run += c;
  }
  state_out[(int64_t)b * state_ld + j] = run;
}

// The selection carry in one pass, for bf16 storage at head dim 64 when the call has key blocks
// enough for a workgroup per CU (many sequences, as in the per-head mode where every head is its own
// sequence, or a long key range, as in the later chunks of a chunked prefill). grid
// (ceil(NKT/(4 KPW)), nseq): wavefront w owns key blocks (4x + w) KPW + u, u < KPW (their K rows in
// registers, one read of each query fragment serving all of them), and the workgroup walks the
// query blocks from the first that can select one of its keys to the last, each staged once into
// LDS by direct loads issued NBUF - 1 blocks ahead (NBUF buffers, one barrier per block), keeping
// each key's running selection in a register. carry[b][rb][j] is stored on entry to block rb (the
// rows before the first block hold the entering value, state_in or zero, as the scan writes them)
// and state_out[b][j] after the last. Each block's sum is block_selection_sum, as in the column-sum
// kernel, and the sums are added in the scan's order: both paths give the same bits, without the
// column sums' round trip through HBM.
//
// Every block issues the same vector-memory operations -- KPW carry stores through a buffer
// resource (lanes that own no key aim past its end, where the store is dropped) and one query-block
// load (past the last block: zero rows into a buffer nobody reads) -- so a fixed count
// vmcnt((NBUF - 2) (KPW + 1)) at the end of a block waits exactly for the next block's load (the
// counter drains in issue order).
constexpr int SEL_CARRY_KPW = 1;             // key blocks per wavefront
constexpr int SEL_CARRY_NBUF = 4;            // query-block buffers
constexpr int SEL_CARRY_MIN_BLOCKS = 256;    // workgroups below which the two-kernel path runs

__global__ __launch_bounds__(NTHREADS) void sel_carry64_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, float* __restrict__ carry,
    const float* state_in, float* state_out, int64_t state_ld, int Tq, int Tk, Strides qs, Strides ks, int q_off,
    int exempt, float scale) {
  using OP = OpBF16;
  using frag = OP::frag;
  constexpr int D = 64, NS = 4, KPW = SEL_CARRY_KPW, NBUF = SEL_CARRY_NBUF, AHEAD = NBUF - 1;
  static_assert(NBUF == 4, "the block loop names four buffers");
  // separate LDS variables, named at compile time, so the compiler knows a block's reads do not
  // touch the buffers the direct loads are filling.
  // Lifetimes (block rb_lo + t lives in buffer t mod 4):
  //   filled: by the direct load g2l_rows64 of every wavefront (a quarter each), for blocks rb_lo,
  //           +1, +2 in the prologue, for block rb + 3 in step t (block rb) -- into the buffer that
  //           held block rb - 1;
  //   drained: by the qa fragment reads of step t only;
  //   separated: the reads of block rb - 1 (step t - 1) from the fill in step t by the end of step
  //           t - 1: lgkmcnt(0) (this wavefront's reads done) and s_barrier (every wavefront's);
  //           the fill of block rb (step t - 3, or the prologue's vmcnt(0)) from its reads by the
  //           vmcnt(4) of step t - 1 (of the 2 per step issued after it, only the last two steps'
  //           may be outstanding) and the same barrier. The peeled last steps keep the count (loads
  //           past the last block read zero rows into buffers nobody reads), and wait_loads() at
  //           the end leaves no load in flight into LDS when the workgroup ends.
  __shared__ __attribute__((aligned(16))) uint16_t sQ0[TILE * D];
  __shared__ __attribute__((aligned(16))) uint16_t sQ1[TILE * D];
  __shared__ __attribute__((aligned(16))) uint16_t sQ2[TILE * D];
  __shared__ __attribute__((aligned(16))) uint16_t sQ3[TILE * D];
  auto sbuf = [&](auto idx) -> uint16_t* {
    constexpr int I = decltype(idx)::value % NBUF;
    if constexpr (I == 0) return sQ0;
    else if constexpr (I == 1) return sQ1;
    else if constexpr (I == 2) return sQ2;
    else return sQ3;
  };
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int NKT = (Tk + TILE - 1) / TILE;
  const int NBq = (Tq + TILE - 1) / TILE;
  const BlockXY bxy = xcd_block();   // each XCD takes whole sequences: their query rows stay in its L2
  const int b = bxy.y;
  const int kb0 = bxy.x * (NWAVES * KPW);
  const uint16_t* q0 = q + qs.at(b, 0);
  const uint16_t* k0 = k + ks.at(b, 0);
  float* plane = carry + (int64_t)b * NBq * Tk;
  const int plane_bytes = NBq * Tk * 4;   // below 2 GiB (the launch checks)
  const __amdgpu_buffer_rsrc_t rs_c = rsrc(plane, plane_bytes);

  // per key block u of the wavefront (blocks past the last one only stage): key j, whether this
  // lane stores key j's values (and the byte offset its stores take: past the plane if not), its
  // K rows, its running selection
  int kb[KPW], jj[KPW], voff[KPW];
  bool owner[KPW];
  frag kf[KPW][NS];
  float run[KPW];
#pragma unroll
  for (int u = 0; u < KPW; ++u) {
    kb[u] = kb0 + wave * KPW + u;
    jj[u] = kb[u] * TILE + n;
    owner[u] = kb[u] < NKT && h == 0 && jj[u] < Tk;
    voff[u] = owner[u] ? jj[u] * 4 : plane_bytes;
#pragma unroll
    for (int s = 0; s < NS; ++s) kf[u][s] = ld_std_bounded<OP>(k0, ks.row, jj[u], Tk, h, s);
    run[u] = (state_in != nullptr && jj[u] < q_off && jj[u] < Tk) ? state_in[(int64_t)b * state_ld + jj[u]] : 0.f;
  }

  // blocks before rb_lo end before the workgroup's first key: no pair of theirs is selectable
  const int lead = kb0 * TILE - q_off;
  const int rb_lo = min(lead > 0 ? lead / TILE : 0, NBq);
#pragma unroll
  for (int u = 0; u < KPW; ++u)
    if (owner[u])
      for (int rb = 0; rb < rb_lo; ++rb) plane[(int64_t)rb * Tk + jj[u]] = run[u];

  const int q_ld = (int)qs.row;
  const __amdgpu_buffer_rsrc_t rs_q = rsrc(q0, (int64_t)Tq * q_ld * 2);   // rows past Tq read zero
  const RowsLane rl_q(q_ld, lane, wave);
  const int nb = NBq - rb_lo;   // blocks walked; block rb_lo + t sits in buffer t mod NBUF
  g2l_rows64(sQ0, rs_q, rl_q, q_ld, rb_lo * TILE, wave);
  g2l_rows64(sQ1, rs_q, rl_q, q_ld, (rb_lo + 1) * TILE, wave);
  g2l_rows64(sQ2, rs_q, rl_q, q_ld, (rb_lo + 2) * TILE, wave);
  wait_loads();
  __syncthreads();

  auto step = [&](int t, auto buf_tag) {
    constexpr int BUF = decltype(buf_tag)::value;
    const int rb = rb_lo + t;
#pragma unroll
    for (int u = 0; u < KPW; ++u)   // the value on entry to the block
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(run[u]), rs_c, voff[u], rb * Tk * 4, 0);
    g2l_rows64(sbuf(std::integral_constant<int, BUF + AHEAD>{}), rs_q, rl_q, q_ld, (rb + AHEAD) * TILE, wave);
    const uint16_t* sQ = sbuf(buf_tag);
    const int qbase = q_off + rb * TILE;
    frag qa[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qa[s] = *reinterpret_cast<const frag*>(sQ + swz64(n, 2 * s + h));
#pragma unroll
    for (int u = 0; u < KPW; ++u) {
      const int kbase = kb[u] * TILE;
      if (kb[u] < NKT && qbase + TILE - 1 > kbase) {
        f32x16 acc = zero16();
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = OP::mma(qa[s], kf[u][s], acc);
        const bool interior = qbase > kbase + TILE - 1 && kbase >= exempt;
        run[u] += block_selection_sum(acc, interior, jj[u] >= exempt ? jj[u] - qbase - 4 * h : 32, scale);
      }
    }
    // The next block's load is in (the loads and stores issued after it may still run), this
    // block's LDS reads are done, then the barrier: as one asm block, since before a compiler-seen
    // barrier the compiler waits for every direct load into LDS, the ones ahead included.
    __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((AHEAD - 1) * (KPW + 1)) : "memory");
  };
  int t = 0;
  for (; t + 3 < nb; t += 4) {
    step(t, std::integral_constant<int, 0>{});
    step(t + 1, std::integral_constant<int, 1>{});
    step(t + 2, std::integral_constant<int, 2>{});
    step(t + 3, std::integral_constant<int, 3>{});
  }
  if (t < nb) step(t, std::integral_constant<int, 0>{});
  if (t + 1 < nb) step(t + 1, std::integral_constant<int, 1>{});
  if (t + 2 < nb) step(t + 2, std::integral_constant<int, 2>{});
  wait_loads();   // nothing may be left in flight into LDS when the workgroup ends
#pragma unroll
  for (int u = 0; u < KPW; ++u)
    if (owner[u]) state_out[(int64_t)b * state_ld + jj[u]] = run[u];
}

// ---------------------------------------------------------------------------------------------
// Forward. grid (ceil(NBq/4), nseq * H/G); wavefront w of block x owns query block
// (gridDim.x-1-x)*4 + w (heavy causal rows launch first) of heads [gi*G, gi*G+G). Key tiles are
// visited newest first, so each row's maximum is usually settled by its diagonal tile and later
// tiles rarely trigger a rescale of the output (skipped when no lane's maximum rises). The next
// tile's K, V^T and carry rows are loaded while the current one is computed (double-buffered LDS).

// Workgroups per CU the forward's register allocation must allow: three at bf16 head dims <= 64
// with one head per wavefront (its LDS fits three), which holds it to 168 registers without spills.
template <class OP, int D, int G>
constexpr int fwd_min_blocks() { return (sizeof(typename OP::elem) == 2 && D <= 64 && G == 1) ? 3 : 1; }

// CV ("contiguous views"): q rows are D apart and its heads Tq * D apart, k rows D apart and its
// heads ks.head apart -- the layout of sa_forward; the view strides are then compile-time facts
// (fewer scalar registers live in the tile loop). Other views take the general instance.
template <class OP, int D, int G, bool CV>
__global__ __launch_bounds__(NTHREADS, (fwd_min_blocks<OP, D, G>())) void fwd_kernel(
    const typename OP::elem* __restrict__ q, const typename OP::elem* __restrict__ k,
    const typename OP::elem* __restrict__ vt, const float* __restrict__ carry,
    float* __restrict__ out, float* __restrict__ rmax, float* __restrict__ rden,
    typename OP::elem* __restrict__ y, Strides ys, int H, int Tq, int Tk, Strides qs, Strides ks, int q_off,
    int64_t ldv, int exempt, float scale, int damp_mode, float train_len) {
  using elem = typename OP::elem;
  using frag = typename OP::frag;
  constexpr int NS = D / OP::KS;          // MFMA steps over D
  constexpr int DB = D / 32;              // 32-row blocks of D
  constexpr int LDK = D + OP::KPAD;
  constexpr int LDV = TILE + OP::TPAD;
  constexpr int AS = OP::acc_steps;
  constexpr int NH = G + 1;
  constexpr int TILE_BYTES = (NH * TILE * LDK + G * D * LDV) * (int)sizeof(elem);
  // two LDS buffers of the key tiles (the next one is written while this one is read) when they fit
  constexpr int NBUF = (2 * TILE_BYTES <= 120 * 1024) ? 2 : 1;

  __shared__ __attribute__((aligned(16))) elem sK[NBUF][NH][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sVt[NBUF][G][D * LDV];
  __shared__ __attribute__((aligned(16))) float sC[NBUF][NWAVES][TILE];   // -carry rows, logit units
  constexpr int LDF = TILE + 4;
  __shared__ __attribute__((aligned(16))) float sF[NWAVES][TILE * LDF];   // each wavefront's F tile
  __shared__ __attribute__((aligned(16))) float sDamp[NWAVES][TILE];      // its queries' damping factors

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int groups = H / G;
  const BlockXY bxy = xcd_block();
  const int b = bxy.y / groups, gi = bxy.y % groups;
  const int hd0 = gi * G;
  const bool has_h0 = (gi == 0);
  const int NBq = (Tq + TILE - 1) / TILE;
  const int NKT = (Tk + TILE - 1) / TILE;
  const int qsb = gridDim.x - 1 - bxy.x;
  const int rb = qsb * NWAVES + wave;
  const int q_rel = rb * TILE + n;
  const int q_abs = q_off + q_rel;
  const int64_t seq_row = (int64_t)b * H;   // row of head 0 of this sequence
  auto q_head = [&](int hh) -> const elem* {
    if constexpr (CV) return q + (seq_row + hh) * Tq * D;
    else return q + qs.at(b, hh);
  };
  auto k_head = [&](int hh) -> const elem* {
    if constexpr (CV) return k + (seq_row + hh) * ks.head;
    else return k + ks.at(b, hh);
  };
  const int64_t q_ld = CV ? (int64_t)D : (int64_t)qs.row;
  const int64_t k_ld = CV ? (int64_t)D : (int64_t)ks.row;

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
    const elem* qh = q_head(hd0 + g);
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[g][s] = ld_std_bounded<OP>(qh, q_ld, q_rel, Tq, h, s);
  }
  if (!has_h0) {
    const elem* qh = q_head(0);
#pragma unroll
    for (int s = 0; s < NS; ++s) q0f[s] = ld_std_bounded<OP>(qh, q_ld, q_rel, Tq, h, s);
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

  // F is kept negated and in units of the unscaled logit q.k (relu(s x) = s relu(x) for s > 0):
  // the logit product then accumulates onto -F and yields q.k - F/s directly, and the scale (with
  // log2 e) enters once, in the exponent's fma.
  const float sl2 = scale * LOG2E;
  const float neg_inv_scale = -1.f / scale;
  float damp = 1.f;
  if (damp_mode != 0) {
    damp = fminf(1.f, train_len / (float)(q_abs + 1));
    if (damp_mode == 2) damp = sqrtf(damp);
  }
  if (lane < TILE) sDamp[wave][lane] = damp;   // (read after the first barrier)

  // Staging of one key tile: K of the group (+ head 0's), V^T of the group, and the carry rows of
  // the workgroup's four query blocks (threads 0..127: wavefront w's row, key tid % 32).
  RowTile<elem, D> nK[NH];
  ColTile<elem, D> nVt[G];
  const elem* k_rows[NH];   // the key rows of this workgroup's heads (outside the tile loop)
#pragma unroll
  for (int g = 0; g < G; ++g) k_rows[g] = k_head(hd0 + g);
  k_rows[G] = k_head(0);
  const int k_ldi = (int)k_ld;
  float nC = 0.f;
  bool nC_ok = false;
  // (every load is unconditional and the loaded values are first used when stored: the vector-
  // memory counter drains in issue order, so a wait inside the tile for one of them, or at a join
  // after a conditional one, would wait for the whole next tile)
  auto load_tile = [&](int kt) {
    const int kbase = kt * TILE;
    const int w = (tid >> 5) & (NWAVES - 1);
    const int rbw = min(qsb * NWAVES + w, NBq - 1);
    const int jj = kbase + (tid & (TILE - 1));
    nC = carry[((int64_t)b * NBq + rbw) * Tk + min(jj, Tk - 1)];   // scaled (zero past the end) when stored
    nC_ok = jj < Tk;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      nK[g].load(k_rows[g], k_ldi, kbase, Tk, tid);
      nVt[g].load(vt + (seq_row + hd0 + g) * D * ldv, ldv, kbase, tid);
    }
    nK[G].load(k_rows[G], k_ldi, kbase, Tk, tid);   // head 0's rows (its own group's copy unused)
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      nK[g].template store<LDK>(sK[buf][g], tid);
      nVt[g].template store_crow<LDV>(sVt[buf][g], tid);
    }
    if (!has_h0) nK[G].template store<LDK>(sK[buf][G], tid);
    if (tid < NWAVES * TILE) sC[buf][tid >> 5][tid & (TILE - 1)] = nC_ok ? nC * neg_inv_scale : 0.f;
  };

  // the next key tile is loaded into registers while this one is computed (stored to the other LDS
  // buffer after it)
  load_tile(wg_end - 1);
  store_tile(0);
  __syncthreads();

  // one key tile; INTERIOR: every key of the tile strictly precedes every query of the workgroup,
  // lies before the end and is not exempt, for every wavefront (straight-line code without masks)
  // DAMP: history damping on (a compile-time fact, so the undamped loops carry no branch for it)
  auto tile_step = [&](int t, auto interior_tag, auto damp_tag) __attribute__((always_inline)) {
    constexpr bool INTERIOR = decltype(interior_tag)::value;
    constexpr bool DAMP = decltype(damp_tag)::value;
    const int kt = wg_end - 1 - t;
    const int buf = NBUF == 2 ? (t & 1) : 0;
    if (t + 1 < wg_end) load_tile(kt - 1);
    if (kt < my_end) {   // (a wavefront past the last query block has none)
      const int kbase = kt * TILE;
      // edge: some key of the tile does not strictly precede every query of the block, lies past
      // the end or is exempt; interior tiles skip the masks (the selection gate is then the logit's
      // sign alone)
      const bool edge =
          !INTERIOR && ((kbase + TILE - 1 >= q_off + rb * TILE) || (kbase + TILE > Tk) || kbase < exempt);
      // (one body for both kinds of tile within a loop: two copies of its accumulating products
      // would make the compiler copy the output sums between register sets every tile)
      auto body = [&]() {
        // Head 0's logits as (queries x keys), lane = key kbase + n: the selection's running sum
        // over queries then stays within the lane. -F (logit units) = -(the carry at the block's
        // first query + the selection by the block's earlier queries); it returns to the
        // (keys x queries) layout of the softmax through this wavefront's LDS rows.
        f32x16 l0t = zero16();
        {
          const elem* k0s = has_h0 ? sK[buf][0] : sK[buf][G];
#pragma unroll
          for (int s = 0; s < NS; ++s)
            l0t = OP::mma(has_h0 ? qf[0][s] : q0f[s], OP::ld_std(k0s, LDK, n, h, s), l0t);
        }
        {
          f32x16 sel;
#pragma unroll
          // -relu as one v_med3 (fminf on a negated value, or a med3 with an infinite bound, which
          // the compiler folds into fminf, would first be canonicalised)
          for (int i = 0; i < 16; ++i) sel[i] = __builtin_amdgcn_fmed3f(-l0t[i], -3.0e38f, 0.f);
          if (edge) {
            // pairs exempt <= j < r; keys past the end and queries past the end hold zero rows
            const int jk = kbase + n;
            const int thr = jk >= exempt ? jk - (q_off + rb * TILE) - 4 * h : 32;
#pragma unroll
            for (int i = 0; i < 16; ++i) sel[i] = crow(i, 0) > thr ? sel[i] : 0.f;
          }
          float run = sC[buf][wave][n];
          float* fw = sF[wave];
#pragma unroll
          for (int a = 0; a < 4; ++a) {
            const Halves g = halves(((sel[4 * a] + sel[4 * a + 1]) + sel[4 * a + 2]) + sel[4 * a + 3]);
            float p = (h == 0) ? run : run + g.lo;   // rows 8a..8a+3 in the low half, 8a+4.. in the high
            float4 dm = make_float4(1.f, 1.f, 1.f, 1.f);   // the rows' damping factors
            if constexpr (DAMP) dm = *reinterpret_cast<const float4*>(&sDamp[wave][8 * a + 4 * h]);
            const float dmv[4] = {dm.x, dm.y, dm.z, dm.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              // a one-head group holding head 0 sends that head's whole adjusted logit,
              // q.k - damp F/s, so its (keys x queries) product is not taken again
              float f = p;
              if (G == 1 && has_h0) f = DAMP ? fmaf(dmv[t], p, l0t[4 * a + t]) : p + l0t[4 * a + t];
              fw[crow(4 * a + t, h) * LDF + n] = f;
              p += sel[4 * a + t];
            }
            run = (run + g.lo) + g.hi;
          }
        }
        lds_wave_sync();
        f32x16 fs;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float4 f4 = *reinterpret_cast<const float4*>(&sF[wave][n * LDF + 8 * a + 4 * h]);
          fs[4 * a] = f4.x;
          fs[4 * a + 1] = f4.y;
          fs[4 * a + 2] = f4.z;
          fs[4 * a + 3] = f4.w;
        }
        if constexpr (DAMP) {
          if (G > 1 || !has_h0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) fs[i] *= damp;
          }
        }

#pragma unroll
        for (int g = 0; g < G; ++g) {
          f32x16 lg = fs;   // the product accumulates onto -F: lg = q.k - F/s
          if (G > 1 || !has_h0) {   // (else head 0's came through LDS whole)
#pragma unroll
            for (int s = 0; s < NS; ++s) lg = OP::mma(OP::ld_std(sK[buf][g], LDK, n, h, s), qf[g][s], lg);
          }
          if (edge) {   // keys j = kbase + crow(i, h) <= min(q_abs, Tk - 1)
            const int thr = min(q_abs, Tk - 1) - kbase - 4 * h;
#pragma unroll
            for (int i = 0; i < 16; ++i) lg[i] = crow(i, 0) <= thr ? lg[i] : -INFINITY;
          }
          float zmax = -INFINITY;
#pragma unroll
          for (int i = 0; i < 16; ++i) zmax = fmaxf(zmax, lg[i]);
          const Halves zh = halves(zmax);
          const float m_new = fmaxf(m[g], fmaxf(zh.lo, zh.hi) * sl2);   // log2 units
          if (__any(m_new > m[g])) {   // some row's maximum rose: rescale what was accumulated
            const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m[g] - m_new);
            m[g] = m_new;
            l[g] *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
              for (int i = 0; i < 16; ++i) o[g][db][i] *= alpha;
          }
          const float mu = (m[g] == -INFINITY) ? 0.f : m[g];   // a row with no key yet
          float psum = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float p = fast_exp2(fmaf(lg[i], sl2, -mu));
            lg[i] = p;
            psum += p;
          }
          l[g] += psum;
          frag pf[AS];
#pragma unroll
          for (int s = 0; s < AS; ++s) pf[s] = OP::from_acc(lg, s);
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int s = 0; s < AS; ++s)
              o[g][db] = OP::mma(OP::ld_perm(sVt[buf][g], LDV, db * 32 + n, h, s), pf[s], o[g][db]);
        }
      };
      body();
    }
    if constexpr (NBUF == 1) __syncthreads();   // the one buffer is free again
    if (t + 1 < wg_end) store_tile(NBUF == 2 ? buf ^ 1 : 0);
    __syncthreads();
  };
  // key tiles newest first: the diagonals and the sequence end, the interior tiles
  // [i_lo, i_hi), then the tiles holding exempt keys
  const int i_lo = min((exempt + TILE - 1) / TILE, wg_end);
  const int i_hi = max(i_lo, min(min(q_off + qsb * NWAVES * TILE, Tk) / TILE, wg_end));
  auto sweep = [&](auto damp_tag) {
    int t = 0;
    for (; t < wg_end - i_hi; ++t) tile_step(t, std::false_type{}, damp_tag);
    for (; t < wg_end - i_lo; ++t) tile_step(t, std::true_type{}, damp_tag);
    for (; t < wg_end; ++t) tile_step(t, std::false_type{}, damp_tag);
  };
  if (damp_mode != 0) sweep(std::true_type{});
  else sweep(std::false_type{});

  if (rb >= NBq || q_rel >= Tq) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const Halves lh = halves(l[g]);
    const float ltot = lh.lo + lh.hi;
    const float inv = 1.f / ltot;
    const int64_t row = (seq_row + hd0 + g) * Tq + q_rel;
    float* orow = out + row * D;
    elem* yrow = y ? y + ys.at(b, hd0 + g) + (int64_t)q_rel * ys.row : nullptr;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        float4 v4 = make_float4(o[g][db][4 * a] * inv, o[g][db][4 * a + 1] * inv,
                                o[g][db][4 * a + 2] * inv, o[g][db][4 * a + 3] * inv);
        const int d = db * 32 + 8 * a + 4 * h;
        *reinterpret_cast<float4*>(orow + d) = v4;
        if (yrow) {
          if constexpr (sizeof(elem) == 2) {
            *reinterpret_cast<uint2*>(yrow + d) = make_uint2(
                (uint32_t)OP::to_elem(v4.x) | ((uint32_t)OP::to_elem(v4.y) << 16),
                (uint32_t)OP::to_elem(v4.z) | ((uint32_t)OP::to_elem(v4.w) << 16));
          } else {
            *reinterpret_cast<float4*>(yrow + d) = v4;
          }
        }
      }
    }
    if (h == 0) {
      rmax[row] = m[g];
      rden[row] = ltot;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Forward, bf16 storage at head dim 64 with G = 2 heads per wavefront or one (odd head counts, the
// per-head mode, grids that fill the CUs only once: fwd64_group): fwd_kernel's tile work with every
// key tile's operands loaded straight into LDS ahead of use (see bwd_kv64_kernel), and the
// selection one tile ahead of the softmax: while tile t's logit products, softmax and value
// products run, the wavefront also takes head 0's logits of tile t + 1 and turns them into that
// tile's F (through its LDS rows, read at the start of tile t + 1), so each tile is one block of
// independent products and arithmetic the compiler interleaves, with no wait inside it for the F
// round trip. A sequence's only head (G = 1, one head) sends its whole adjusted logits through the
// LDS rows instead (as fwd_kernel does), so it takes one logit product per tile. The K rows of the
// group's heads (swz64) and their V rows (swzq, read transposed by the value products, get_trq)
// load one tile ahead into two buffers; head 0's K rows and each wavefront's carry row two tiles
// ahead into two more; all four are separate LDS variables and the tile loop runs in pairs, so
// every access names its buffer at compile time; one barrier per tile. Two workgroups per CU at
// G = 2, three at G = 1.

template <int G>
struct FwdTileBuf64 {
  __attribute__((aligned(16))) uint16_t k[G][TILE * 64];   // K rows of the group's heads
  __attribute__((aligned(16))) uint16_t v[G][TILE * 64];   // their V rows
};
struct FwdSelBuf64 {
  __attribute__((aligned(16))) uint16_t k0[TILE * 64];      // head 0's K rows
  __attribute__((aligned(16))) float c[NWAVES][64];         // per wavefront: the carry of each key
};

template <bool CV, int G>   // CV: as fwd_kernel; G: heads per wavefront (1 or 2)
__global__ __launch_bounds__(NTHREADS, G == 1 ? 3 : 2) void fwd64_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ carry, float* __restrict__ out, float* __restrict__ rmax, float* __restrict__ rden,
    uint16_t* __restrict__ y, Strides ys, int H, int Tq, int Tk, Strides qs, Strides ks, Strides vs, int q_off,
    int exempt, float scale, int damp_mode, float train_len) {
  using OP = OpBF16;
  using elem = uint16_t;
  using frag = OP::frag;
  constexpr int D = 64, NS = 4, DB = 2, AS = 2;
  static_assert(G == 1 || G == 2, "one or two heads per wavefront");
  // LDS lifetimes (tile t = key tile wg_end - 1 - t; every fill is a direct load of all four
  // wavefronts, a quarter each, and each tile step ends with wait_loads() -- this wavefront's loads
  // have landed -- and __syncthreads() -- every wavefront's have, and every wavefront is past its
  // reads of the step):
  //   sB0, sB1  tile t's K and V rows, buffer t mod 2. Filled: the prologue (tile 0), tile step
  //             t - 1 (tile t). Drained: tile step t (the logit and value products). Separated:
  //             the last reads of buffer t mod 2 (tile step t - 2) from its fill (tile step t - 1)
  //             by the end of tile step t - 2.
  //   sS0, sS1  tile t's head-0 K rows and each wavefront's carry row, buffer t mod 2. Filled: the
  //             prologue (tiles 0, 1), tile step t - 2 (tile t). Drained: the selection of tile t
  //             (select(), run at the end of tile step t - 1; tile 0's in the sweep's prologue).
  //             Separated: the selection of tile t - 2 (end of tile step t - 3) from the fill in tile
  //             step t - 2 by the end of tile step t - 3; tile 0's selection from tile 2's fill (tile
  //             step 0) by the barrier after it in the sweep's prologue; the fill of tile t (tile
  //             step t - 2) from its selection (end of tile step t - 1) by the end of tile step t - 2.
  //   sF        per wavefront, its F tile: written by select() of tile t + 1 at the end of tile step t
  //             (transposing stores), read at the start of tile step t + 1; the same wavefront's
  //             writes follow its reads of tile t in program order, and the reads of tile t + 1 follow
  //             the writes across the step's barrier.
  //   sDamp     per wavefront, its queries' damping factors: written once before the prologue's
  //             barrier, read only after it.
  __shared__ FwdTileBuf64<G> sB0, sB1;   // tile t's K and V rows in buffer t mod 2
  __shared__ FwdSelBuf64 sS0, sS1;    // tile t's head-0 K rows and carry rows in buffer t mod 2
  constexpr int LDF = TILE + 4;
  __shared__ __attribute__((aligned(16))) float sF[NWAVES][TILE * LDF];   // each wavefront's F tile
  __shared__ __attribute__((aligned(16))) float sDamp[NWAVES][TILE];      // its queries' damping factors

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int groups = H / G;
  const BlockXY bxy = part_block();
  const int b = bxy.y / groups, gi = bxy.y % groups;
  const int hd0 = gi * G;
  const bool has_h0 = (gi == 0);
  // Head 0's adjusted logits come through LDS whole when it is the sequence's only head (one product
  // per tile instead of two). With other heads beside it, head 0 takes the path of every head (its
  // product accumulating onto -F), so one and two heads per wavefront give the same bits and the
  // host may choose either per launch.
  const bool whole = G == 1 && has_h0 && H == 1;
  const int NBq = (Tq + TILE - 1) / TILE;
  const int NKT = (Tk + TILE - 1) / TILE;
  const int qsb = gridDim.x - 1 - bxy.x;
  const int rb = qsb * NWAVES + wave;
  const int q_rel = rb * TILE + n;
  const int q_abs = q_off + q_rel;
  const int64_t seq_row = (int64_t)b * H;
  auto q_head = [&](int hh) -> const elem* {
    if constexpr (CV) return q + (seq_row + hh) * Tq * D;
    else return q + qs.at(b, hh);
  };
  auto k_head = [&](int hh) -> const elem* {
    if constexpr (CV) return k + (seq_row + hh) * ks.head;
    else return k + ks.at(b, hh);
  };
  const int64_t q_ld = CV ? (int64_t)D : (int64_t)qs.row;
  const int k_ld = CV ? D : (int)ks.row;

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
    const elem* qh = q_head(hd0 + g);
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[g][s] = ld_std_bounded<OP>(qh, q_ld, q_rel, Tq, h, s);
  }
  if (!has_h0) {
    const elem* qh = q_head(0);
#pragma unroll
    for (int s = 0; s < NS; ++s) q0f[s] = ld_std_bounded<OP>(qh, q_ld, q_rel, Tq, h, s);
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
  // F negated, in units of the unscaled logit q.k (see fwd_kernel)
  const float sl2 = scale * LOG2E;
  const float neg_inv_scale = -1.f / scale;
  float damp = 1.f;
  if (damp_mode != 0) {
    damp = fminf(1.f, train_len / (float)(q_abs + 1));
    if (damp_mode == 2) damp = sqrtf(damp);
  }
  if (lane < TILE) sDamp[wave][lane] = damp;   // (read after the first barrier)

  // key-side sources and this lane's parts of the direct loads
  const __amdgpu_buffer_rsrc_t rs_k0 = rsrc(k_head(hd0), (int64_t)Tk * k_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_k1 = rsrc(k_head(hd0 + G - 1), (int64_t)Tk * k_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_kh = rsrc(k_head(0), (int64_t)Tk * k_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_v0 = rsrc(v + vs.at(b, hd0), (int64_t)Tk * vs.row * 2);
  const __amdgpu_buffer_rsrc_t rs_v1 = rsrc(v + vs.at(b, hd0 + G - 1), (int64_t)Tk * vs.row * 2);
  // this wavefront's carry row (its query block's; keys past the end read zero)
  const __amdgpu_buffer_rsrc_t rs_c =
      rsrc(carry + ((int64_t)b * NBq + min(rb, NBq - 1)) * Tk, (int64_t)Tk * 4);
  const RowsLane rl_k(k_ld, lane, wave);
  const RowsLaneQ rl_v(vs.row, lane, wave);

  // key tile kt's K and V rows (into B), and its head-0 K rows and carry rows (into S), by direct
  // loads only
  auto load_tile = [&](int kt, FwdTileBuf64<G>& B) {
    const int kbase = kt * TILE;
    g2l_rows64(B.k[0], rs_k0, rl_k, k_ld, kbase, wave);
    g2l_rowsq(B.v[0], rs_v0, rl_v, vs.row, kbase, wave);
    if constexpr (G == 2) {
      g2l_rows64(B.k[1], rs_k1, rl_k, k_ld, kbase, wave);
      g2l_rowsq(B.v[1], rs_v1, rl_v, vs.row, kbase, wave);
    }
  };
  auto load_sel = [&](int kt, FwdSelBuf64& S) {
    const int kbase = kt * TILE;
    g2l_rows64(S.k0, rs_kh, rl_k, k_ld, kbase, wave);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_c, lds_ptr(S.c[wave]), 4, (kbase + n) * 4, 0, 0, 0);
  };
  auto rfrag = [&](const elem* tile, int s) -> frag {
    return *reinterpret_cast<const frag*>(tile + swz64(n, 2 * s + h));
  };

  // Key tile kt's selection: head 0's logits as (queries x keys), lane = key, so the running sum over
  // queries stays within the lane; -F (logit units) = -(the carry at the block's first query + the
  // selection by the block's earlier queries) goes to this wavefront's LDS rows, where the tile's
  // softmax reads it in the (keys x queries) layout (with `whole`: q.k - damp F/s, damping per row).
  auto select = [&](int kt, const FwdSelBuf64& S, auto damp_tag) {
    constexpr bool DAMP = decltype(damp_tag)::value;
    const int kbase = kt * TILE;
    f32x16 l0t = zero16();
#pragma unroll
    for (int s = 0; s < NS; ++s) l0t = OP::mma(has_h0 ? qf[0][s] : q0f[s], rfrag(S.k0, s), l0t);
    f32x16 sel;
    // -relu as one v_med3 (see fwd_kernel)
#pragma unroll
    for (int i = 0; i < 16; ++i) sel[i] = __builtin_amdgcn_fmed3f(-l0t[i], -3.0e38f, 0.f);
    const bool edge = (kbase + TILE - 1 >= q_off + rb * TILE) || (kbase + TILE > Tk) || kbase < exempt;
    if (edge) {
      // pairs exempt <= j < r; keys past the end and queries past the end hold zero rows
      const int jk = kbase + n;
      const int thr = jk >= exempt ? jk - (q_off + rb * TILE) - 4 * h : 32;
#pragma unroll
      for (int i = 0; i < 16; ++i) sel[i] = crow(i, 0) > thr ? sel[i] : 0.f;
    }
    float run = S.c[wave][n] * neg_inv_scale;
    float* fw = sF[wave];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const Halves g = halves(((sel[4 * a] + sel[4 * a + 1]) + sel[4 * a + 2]) + sel[4 * a + 3]);
      float p = (h == 0) ? run : run + g.lo;
      float4 dm = make_float4(1.f, 1.f, 1.f, 1.f);   // the rows' damping factors
      if constexpr (DAMP && G == 1) dm = *reinterpret_cast<const float4*>(&sDamp[wave][8 * a + 4 * h]);
      const float dmv[4] = {dm.x, dm.y, dm.z, dm.w};
#pragma unroll
      for (int t2 = 0; t2 < 4; ++t2) {
        float f = p;
        if (whole) f = DAMP ? fmaf(dmv[t2], p, l0t[4 * a + t2]) : p + l0t[4 * a + t2];
        fw[crow(4 * a + t2, h) * LDF + n] = f;
        p += sel[4 * a + t2];
      }
      run = (run + g.lo) + g.hi;
    }
  };

  // the first tile's operands, head-0 rows and carry of the first two (its F at the sweep's start)
  load_tile(wg_end - 1, sB0);
  load_sel(wg_end - 1, sS0);
  if (wg_end >= 2) load_sel(wg_end - 2, sS1);
  wait_loads();
  __syncthreads();

  // tile t (buffer t mod 2, named by ODD); INTERIOR and DAMP as in fwd_kernel (INTERIOR for tile t;
  // the selection of tile t + 1 checks its own tile)
  auto tile_step = [&](int t, auto interior_tag, auto damp_tag, auto odd_tag) __attribute__((always_inline)) {
    constexpr bool INTERIOR = decltype(interior_tag)::value;
    constexpr bool DAMP = decltype(damp_tag)::value;
    constexpr bool ODD = decltype(odd_tag)::value;
    FwdTileBuf64<G>& B = ODD ? sB1 : sB0;
    const int kt = wg_end - 1 - t;
    // free since the last barrier: the other tile buffer, and this parity's head-0 buffer (tile t's
    // rows were used by the selection of tile t during tile t - 1)
    if (t + 1 < wg_end) load_tile(kt - 1, ODD ? sB0 : sB1);
    if (t + 2 < wg_end) load_sel(kt - 2, ODD ? sS1 : sS0);
    if (kt < my_end) {   // (a wavefront past the last query block has none)
      const int kbase = kt * TILE;
      const bool edge =
          !INTERIOR && ((kbase + TILE - 1 >= q_off + rb * TILE) || (kbase + TILE > Tk) || kbase < exempt);
      f32x16 fs;   // -F of this tile, written by its selection
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float4 f4 = *reinterpret_cast<const float4*>(&sF[wave][n * LDF + 8 * a + 4 * h]);
        fs[4 * a] = f4.x;
        fs[4 * a + 1] = f4.y;
        fs[4 * a + 2] = f4.z;
        fs[4 * a + 3] = f4.w;
      }
      if constexpr (DAMP) {
        if (!whole) {
#pragma unroll
          for (int i = 0; i < 16; ++i) fs[i] *= damp;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        f32x16 lg = fs;   // the product accumulates onto -F: lg = q.k - F/s
        if (!whole) {
#pragma unroll
          for (int s = 0; s < NS; ++s) lg = OP::mma(rfrag(B.k[g], s), qf[g][s], lg);
        }
        if (edge) {
          const int thr = min(q_abs, Tk - 1) - kbase - 4 * h;
#pragma unroll
          for (int i = 0; i < 16; ++i) lg[i] = crow(i, 0) <= thr ? lg[i] : -INFINITY;
        }
        float zmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) zmax = fmaxf(zmax, lg[i]);
        const Halves zh = halves(zmax);
        const float m_new = fmaxf(m[g], fmaxf(zh.lo, zh.hi) * sl2);
        if (__any(m_new > m[g])) {
          const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m[g] - m_new);
          m[g] = m_new;
          l[g] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[g][db][i] *= alpha;
        }
        const float mu = (m[g] == -INFINITY) ? 0.f : m[g];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = fast_exp2(fmaf(lg[i], sl2, -mu));
          lg[i] = p;
          psum += p;
        }
        l[g] += psum;
        frag pf[AS];
#pragma unroll
        for (int s = 0; s < AS; ++s) pf[s] = OP::from_acc(lg, s);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int s = 0; s < AS; ++s)
            o[g][db] = OP::mma(get_trq<true>(B.v[g], lane, db, s), pf[s], o[g][db]);
      }
    }
    // the next tile's F (after this tile's reads of the wavefront's F rows, in program order)
    if (t + 1 < wg_end && kt - 1 < my_end) select(kt - 1, ODD ? sS0 : sS1, damp_tag);
    wait_loads();
    __syncthreads();   // the next tile's operands are in; every wavefront is done with this one
  };
  const int i_lo = min((exempt + TILE - 1) / TILE, wg_end);
  const int i_hi = max(i_lo, min(min(q_off + qsb * NWAVES * TILE, Tk) / TILE, wg_end));
  auto sweep = [&](auto damp_tag) {
    if (wg_end - 1 < my_end) select(wg_end - 1, sS0, damp_tag);   // the first tile's F
    // The first tile step loads tile 2's head-0 K rows into sS0, whose rows every wavefront has
    // just read for that F: all of them must be past their reads first.
    __syncthreads();
    auto run = [&](int t0, int t1, auto interior_tag) {
      int t = t0;
      if (t < t1 && (t & 1)) tile_step(t++, interior_tag, damp_tag, std::true_type{});
      for (; t + 1 < t1; t += 2) {
        tile_step(t, interior_tag, damp_tag, std::false_type{});
        tile_step(t + 1, interior_tag, damp_tag, std::true_type{});
      }
      if (t < t1) tile_step(t, interior_tag, damp_tag, std::false_type{});
    };
    run(0, wg_end - i_hi, std::false_type{});
    run(wg_end - i_hi, wg_end - i_lo, std::true_type{});
    run(wg_end - i_lo, wg_end, std::false_type{});
  };
  if (damp_mode != 0) sweep(std::true_type{});
  else sweep(std::false_type{});

  if (rb >= NBq || q_rel >= Tq) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const Halves lh = halves(l[g]);
    const float ltot = lh.lo + lh.hi;
    const float inv = 1.f / ltot;
    const int64_t row = (seq_row + hd0 + g) * Tq + q_rel;
    float* orow = out + row * D;
    elem* yrow = y ? y + ys.at(b, hd0 + g) + (int64_t)q_rel * ys.row : nullptr;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        float4 v4 = make_float4(o[g][db][4 * a] * inv, o[g][db][4 * a + 1] * inv, o[g][db][4 * a + 2] * inv,
                                o[g][db][4 * a + 3] * inv);
        const int d = db * 32 + 8 * a + 4 * h;
        *reinterpret_cast<float4*>(orow + d) = v4;
        if (yrow)
          *reinterpret_cast<uint2*>(yrow + d) =
              make_uint2((uint32_t)OP::to_elem(v4.x) | ((uint32_t)OP::to_elem(v4.y) << 16),
                         (uint32_t)OP::to_elem(v4.z) | ((uint32_t)OP::to_elem(v4.w) << 16));
      }
    }
    if (h == 0) {
      rmax[row] = m[g];
      rden[row] = ltot;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward preparation: lse = rmax + log2(rden), ndbar = -rowsum(dO * O) (negated: the dO.v
// products accumulate onto it), and, except at bf16 head dim 64 (whose kernels read the rows
// transposed from LDS), the transposed copies Q^T, dO^T, K^T (R, D, ldt). The
// statistics are laid out (R, ldt), each head's rows padded to ldt with lse = +inf (P = 0) and
// ndbar = 0, so a 32-row tile of them is always in bounds; they take D/8 lanes per row (8 elements
// each, so the loads of a row are contiguous across its lanes); transposes go by tiles.

template <class OP, int D>
__global__ __launch_bounds__(NTHREADS) void bwd_rowstats_kernel(
    const typename OP::elem* __restrict__ dout, Strides dos, int H, int T, const float* __restrict__ out,
    const float* __restrict__ rmax, const float* __restrict__ rden,
    float* __restrict__ lse, float* __restrict__ ndbar, int64_t ldt, int64_t rows) {
  using elem = typename OP::elem;
  constexpr int LPR = D / 8;   // lanes per row
  const int64_t g = (int64_t)blockIdx.x * NTHREADS + threadIdx.x;
  const int64_t pr = g / LPR;   // padded row: head pr / ldt, row t
  const int part = (int)(g % LPR);
  const int64_t hr = pr / ldt;   // b * H + head
  const int t = (int)(pr - hr * ldt);
  const int64_t r = hr * T + t;
  float acc = 0.f;
  if (pr < rows && t < T) {
    const elem* dr = dout + dos.at(hr / H, hr % H) + (int64_t)t * dos.row + part * 8;
    const float* orow = out + r * D + part * 8;
    const float4 o0 = *reinterpret_cast<const float4*>(orow);
    const float4 o1 = *reinterpret_cast<const float4*>(orow + 4);
    const float ov[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
    elem dv[8];
    if constexpr (sizeof(elem) == 2) {
      *reinterpret_cast<uint4*>(dv) = *reinterpret_cast<const uint4*>(dr);
    } else {
      *reinterpret_cast<float4*>(dv) = *reinterpret_cast<const float4*>(dr);
      *reinterpret_cast<float4*>(dv + 4) = *reinterpret_cast<const float4*>(dr + 4);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += OP::to_float(dv[e]) * ov[e];
  }
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (pr < rows && part == 0) {
    ndbar[pr] = t < T ? -acc : 0.f;
    lse[pr] = t < T ? rmax[r] + __log2f(rden[r]) : INFINITY;
  }
}

// in (R = nseq * H views of T rows, Strides is) -> outT (R, D, ldt), zero past T; a workgroup moves
// a [64 t][D] slab through LDS in 16-byte chunks: row chunks in, then 8 (bf16) or 4 (fp32)
// consecutive t of one d out.
template <typename E, int D>
__global__ __launch_bounds__(NTHREADS) void transpose_kernel(const E* __restrict__ in, E* __restrict__ outT,
                                                             int T, int64_t ldt, Strides is, int H) {
  constexpr int EPC = 16 / (int)sizeof(E);
  constexpr int LDS_LD = D + EPC;   // padded row: 16-byte aligned, rows on shifted banks
  __shared__ __attribute__((aligned(16))) E tile[64 * LDS_LD];
  const int64_t r = blockIdx.y;
  const int t0 = blockIdx.x * 64;
  const E* src = in + is.at(r / H, r % H);
  for (int c = threadIdx.x; c < 64 * D / EPC; c += NTHREADS) {
    const int tt = c / (D / EPC), d0 = (c % (D / EPC)) * EPC;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (t0 + tt < T) v = *reinterpret_cast<const uint4*>(src + (int64_t)(t0 + tt) * is.row + d0);
    *reinterpret_cast<uint4*>(&tile[tt * LDS_LD + d0]) = v;
  }
  __syncthreads();
  E* dst = outT + r * D * ldt;
  for (int c = threadIdx.x; c < D * 64 / EPC; c += NTHREADS) {
    const int d = c % D, tt0 = (c / D) * EPC;
    union {
      uint4 v;
      E e[EPC];
    } u;
#pragma unroll
    for (int e = 0; e < EPC; ++e) u.e[e] = tile[(tt0 + e) * LDS_LD + d];
    if (t0 + tt0 < ldt) *reinterpret_cast<uint4*>(dst + (int64_t)d * ldt + t0 + tt0) = u.v;
  }
}

// The same transpose for 2-byte elements without LDS: a thread moves one 8 x 8 block (8 t, 8 d) --
// eight 16-byte row loads (t past T read as zero), the block transposed in registers (each output
// word joins the same half-word of two rows), eight 16-byte column stores. A wavefront's loads and
// stores cover whole 128-byte segments (eight lanes per row or column).
template <int D>
__global__ __launch_bounds__(NTHREADS) void transpose8_kernel(const uint16_t* __restrict__ in,
                                                              uint16_t* __restrict__ outT, int T, int64_t ldt,
                                                              Strides is, int H) {
  constexpr int CB = D / 8;   // 8-column blocks per row
  const int64_t r = blockIdx.y;
  const int c = threadIdx.x % CB;
  const int64_t t0 = ((int64_t)blockIdx.x * (NTHREADS / CB) + threadIdx.x / CB) * 8;
  if (t0 >= ldt) return;
  const uint16_t* src = in + is.at(r / H, r % H) + 8 * c;
  uint4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    v[k] = (t0 + k < T) ? *reinterpret_cast<const uint4*>(src + (t0 + k) * is.row) : make_uint4(0u, 0u, 0u, 0u);
  auto word = [&](int k, int w) -> uint32_t {
    return w == 0 ? v[k].x : (w == 1 ? v[k].y : (w == 2 ? v[k].z : v[k].w));
  };
  uint16_t* dst = outT + r * D * ldt + t0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t lo = word(2 * w, e >> 1), hi = word(2 * w + 1, e >> 1);
      o[w] = (e & 1) ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
    }
    *reinterpret_cast<uint4*>(dst + (int64_t)(8 * c + e) * ldt) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// in (R views, Strides is) -> outT (R, D, ldt), ldt a multiple of 64, zero past T.
template <typename E, int D>
void launch_transpose(const E* in, E* outT, int T, int64_t ldt, const Strides& is, int H, int64_t R,
                      hipStream_t st) {
  if constexpr (sizeof(E) == 2) {
    constexpr int rows_per_block = NTHREADS / (D / 8) * 8;
    const dim3 grid((unsigned)cdiv(ldt, rows_per_block), (unsigned)R);
    hipLaunchKernelGGL((transpose8_kernel<D>), grid, dim3(NTHREADS), 0, st, reinterpret_cast<const uint16_t*>(in),
                       reinterpret_cast<uint16_t*>(outT), T, ldt, is, H);
  } else {
    hipLaunchKernelGGL((transpose_kernel<E, D>), dim3((unsigned)cdiv(ldt, 64), (unsigned)R), dim3(NTHREADS), 0, st,
                       in, outT, T, ldt, is, H);
  }
}

// ---------------------------------------------------------------------------------------------
// Backward kernel shapes of the generic instances (every storage type and head dim but bf16 at 64,
// which bwd_kv64_kernel / bwd_dq64_kernel take): each tile is loaded into registers, stored to LDS
// and computed in turn (one LDS buffer), the load latency left to the CU's other workgroup. Both
// sides fit two workgroups per CU at bf16 head dims <= 64: the key side's K and V rows sit in LDS,
// the query side's Q and dO rows and row statistics in registers.
template <class OP, int D>
constexpr int dq_min_blocks() { return (sizeof(typename OP::elem) == 2 && D <= 64) ? 2 : 1; }
template <class OP, int D, int G>
constexpr int kv_min_blocks() { return (sizeof(typename OP::elem) == 2 && D <= 64 && G == 1) ? 2 : 1; }

// ---------------------------------------------------------------------------------------------
// Gradient stores to a caller's view (fp32 or bf16 elements): one element, or four consecutive
// elements of a row (d a multiple of 4; the views' rows start 16-byte aligned).
__device__ __forceinline__ void store_grad1(const GradView& v, int64_t b, int hh, int row, int d, float x) {
  const int64_t o = v.s.at(b, hh) + (int64_t)row * v.s.row + d;
  if (v.f32) static_cast<float*>(v.p)[o] = x;
  else static_cast<uint16_t*>(v.p)[o] = OpBF16::to_elem(x);
}
__device__ __forceinline__ void store_grad4(const GradView& v, int64_t b, int hh, int row, int d, float4 x) {
  const int64_t o = v.s.at(b, hh) + (int64_t)row * v.s.row + d;
  if (v.f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(v.p) + o) = x;
  } else {
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(v.p) + o) =
        make_uint2((uint32_t)OpBF16::to_elem(x.x) | ((uint32_t)OpBF16::to_elem(x.y) << 16),
                   (uint32_t)OpBF16::to_elem(x.z) | ((uint32_t)OpBF16::to_elem(x.w) << 16));
  }
}

// ---------------------------------------------------------------------------------------------
// Backward helpers on (queries x keys) C-layout tiles: lane n holds key j = key0 + n, rows are the
// queries qbase + crow(i, h), i = 0..15 (h = lane / 32).

// Backward tiles hold (queries x keys) in C layout: lane n is key j, element i is query row
// qbase + crow(i, h). Rows past the sequence end need no mask here: their Q, dO rows are staged as
// zeros and their lse as +inf, so their logits, selection, P and dz are all zero. The remaining
// masks compare the row's offset within its half-wavefront, crow(i, 0), with a per-lane threshold:
//   P, dz:     j <= r  (and j < T)           <=>  crow(i, 0) >= thr_p = j - qbase - 4h  (32 if j >= T)
//   selection: j <  r  (and exempt <= j < T) <=>  crow(i, 0) >  thr_s = j - qbase - 4h  (32 if not)
struct TileMasks {
  int thr_p, thr_s;
  __device__ __forceinline__ TileMasks(int j, int qbase, int T, int exempt, int h) {
    const int d = j - qbase - 4 * h;
    thr_p = j < T ? d : 32;
    thr_s = (j < T && j >= exempt) ? d : 32;
  }
};

// Head 0's selection on a tile of its raw logits l0 = q.k, in the same unscaled units (relu(s x) =
// s relu(x) for s > 0): sel = relu(l0) where exempt <= j < r < T, and the negated history
// fs[r, j] = nhist - sum of sel over the tile's earlier rows, nhist = -(the selection before the
// tile) / s (the running sum runs down the rows; the half-wavefronts exchange partial sums). A
// logit product accumulating onto fs then yields q.k - F/s. Bit i of gate is sel[i] > 0, the gate
// of the gradient path. `edge` (wave-uniform) marks tiles where some pair fails exempt <= j < r:
// the mask is applied there (every tile when ALWAYS, which costs a few instructions per element
// but no branch).
template <bool ALWAYS>
__device__ __forceinline__ void selection_tile(const f32x16& l0, float nhist, int h, bool edge,
                                               const TileMasks& mk, uint32_t& gate, f32x16& fs) {
  f32x16 sel;
  // relu as one v_med3 (fmaxf on a product's result would first be canonicalised)
#pragma unroll
  for (int i = 0; i < 16; ++i) sel[i] = __builtin_amdgcn_fmed3f(l0[i], 0.f, 3.0e38f);
  if (ALWAYS || edge) {
#pragma unroll
    for (int i = 0; i < 16; ++i) sel[i] = crow(i, 0) > mk.thr_s ? sel[i] : 0.f;
  }
  gate = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) gate |= sel[i] > 0.f ? (1u << i) : 0u;
  float run = nhist;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const Halves g = halves(((sel[4 * a] + sel[4 * a + 1]) + sel[4 * a + 2]) + sel[4 * a + 3]);
    float p = (h == 0) ? run : run - g.lo;   // rows 8a..8a+3 sit in the low half, 8a+4.. in the high
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      fs[4 * a + t] = p;
      p -= sel[4 * a + t];
    }
    run = (run - g.lo) - g.hi;
  }
}

// Selection gradient path: U[r, j] = u_in + sum of z over the tile's later rows, and
// g = -U where the gate is set, else 0. Returns u_in + the sum over the whole tile (U entering the
// tile above). The sum runs negated so the select takes -U without a modifier.
__device__ __forceinline__ float gpath_tile(const f32x16& z, float u_in, uint32_t gate, int h, f32x16& gp) {
  float nrun = -u_in;
#pragma unroll
  for (int a = 3; a >= 0; --a) {
    const Halves g = halves(((z[4 * a + 3] + z[4 * a + 2]) + z[4 * a + 1]) + z[4 * a]);
    float np = (h == 1) ? nrun : nrun - g.hi;
#pragma unroll
    for (int t = 3; t >= 0; --t) {
      const int i = 4 * a + t;
      gp[i] = ((gate >> i) & 1u) ? np : 0.f;
      np -= z[i];
    }
    nrun = (nrun - g.hi) - g.lo;
  }
  return -nrun;
}

// P = exp2(s log2e lg - lse) and dz = P dpb on a tile, lg = q.k - F/s, dpb = dO.v - dbar (the
// product accumulated onto -dbar); lse of the tile's rows comes from LDS (4 consecutive rows per
// float4). Pairs outside j <= r, j < T are zeroed on `edge` tiles (every tile when ALWAYS).
template <bool ALWAYS>
__device__ __forceinline__ void p_dz_tile(const f32x16& lg, const f32x16& dpb, const float* slse, float sl2,
                                          int h, bool edge, const TileMasks& mk, f32x16& pr, f32x16& dz) {
  if constexpr (ALWAYS) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float4 ls = *reinterpret_cast<const float4*>(slse + 8 * a + 4 * h);
      const float lsv[4] = {ls.x, ls.y, ls.z, ls.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int i = 4 * a + t;
        const float p = fast_exp2(fmaf(lg[i], sl2, -lsv[t]));
        pr[i] = crow(i, 0) >= mk.thr_p ? p : 0.f;
        dz[i] = pr[i] * dpb[i];
      }
    }
  } else {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float4 ls = *reinterpret_cast<const float4*>(slse + 8 * a + 4 * h);
      const float lsv[4] = {ls.x, ls.y, ls.z, ls.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) pr[4 * a + t] = fast_exp2(fmaf(lg[4 * a + t], sl2, -lsv[t]));
    }
    if (edge) {
#pragma unroll
      for (int i = 0; i < 16; ++i) pr[i] = crow(i, 0) >= mk.thr_p ? pr[i] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) dz[i] = pr[i] * dpb[i];
  }
}

// p_dz_tile with the rows' lse values already in registers (element i: row crow(i, h)).
__device__ __forceinline__ void p_dz_tile_r(const f32x16& lg, const f32x16& dpb, const f32x16& lsev, float sl2,
                                            bool edge, const TileMasks& mk, f32x16& pr, f32x16& dz) {
#pragma unroll
  for (int i = 0; i < 16; ++i) pr[i] = fast_exp2(fmaf(lg[i], sl2, -lsev[i]));
  if (edge) {
#pragma unroll
    for (int i = 0; i < 16; ++i) pr[i] = crow(i, 0) >= mk.thr_p ? pr[i] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) dz[i] = pr[i] * dpb[i];
}

// Whether some value of the wavefront's tile is large enough for the split-operand products (the
// rounding of a bf16 operand then matters beside the others): g sums dz over every later query of
// the group's heads and can outgrow the dz tiles many times. Taken on g, and on head 0's dz + g.
__device__ __forceinline__ bool big_tile(const f32x16& x) {
  bool big = false;
#pragma unroll
  for (int i = 0; i < 16; ++i) big |= fabsf(x[i]) > 0.25f;
  return __any(big);
}

// ---------------------------------------------------------------------------------------------
// Backward, key side. grid (ceil(T/128), nseq * H/G); wavefront w owns keys [x*128 + 32w, +32) of
// heads [gi*G, gi*G+G) and sweeps the query tiles last to first, with K, V and the dK, dV sums in
// registers. The selection suffix U (over this group's heads) is checkpointed on entry to every
// query tile, for the dQ kernel, into row qb (keys j < 32 (qb + 1)) of the (gi, b) plane of ucheck,
// a lower-triangular plane of rows laid end to end (utri_row). Head 0's dK gets g = -gate*U from every
// group: the group holding head 0 folds it into head 0's dz; the others add their share to dk0x.

// CV: every view is the contiguous (nseq, H, T, D) layout of sa_backward (see fwd_kernel).
template <class OP, int D, int G, bool CV>
__global__ __launch_bounds__(NTHREADS, (kv_min_blocks<OP, D, G>())) void bwd_kv_kernel(
    const typename OP::elem* __restrict__ q, const typename OP::elem* __restrict__ k,
    const typename OP::elem* __restrict__ v, const typename OP::elem* __restrict__ qt,
    const typename OP::elem* __restrict__ dout, const typename OP::elem* __restrict__ dot, Strides qs,
    Strides ks, Strides vs, Strides dos, const float* __restrict__ lse, const float* __restrict__ dbar,
    const float* __restrict__ carry, float* __restrict__ ucheck, float* __restrict__ dk0h, float* __restrict__ dk0x,
    GradView dkv, GradView dvv, int nseq, int H, int T, int64_t ldt, int exempt, float scale) {
  using elem = typename OP::elem;
  using frag = typename OP::frag;
  constexpr int NS = D / OP::KS;
  constexpr int DB = D / 32;
  constexpr int LDK = D + OP::KPAD;
  constexpr int LDV = TILE + OP::TPAD;
  constexpr int AS = OP::acc_steps;
  constexpr int NH = G + 1;   // staged heads: the group, then head 0 when outside the group
  constexpr int TILE_BYTES = (NH * (TILE * LDK + D * LDV) + G * (TILE * LDK + D * LDV)) * (int)sizeof(elem);

  __shared__ __attribute__((aligned(16))) elem sQ[NH][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sQt[NH][D * LDV];
  __shared__ __attribute__((aligned(16))) elem sdO[G][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sdOt[G][D * LDV];
  __shared__ __attribute__((aligned(16))) float sLse[G][TILE];
  __shared__ __attribute__((aligned(16))) float sDb[G][TILE];
  // Each wavefront's K and V rows are read from LDS per tile instead of being held in registers,
  // when they fit unpadded (swz64) beside the query tiles in half the CU's LDS: the registers they
  // free let two workgroups share a CU. Head 0's K rows (for a group without head 0) stay in
  // registers.
  constexpr int NKV = 2 * G;   // K, V of each head of the group
  constexpr int OTHER_LDS = TILE_BYTES + 2 * G * TILE * 4;
  constexpr bool KVLDS = sizeof(elem) == 2 && D == 64 && OTHER_LDS + NWAVES * NKV * TILE * D * 2 <= 80 * 1024;
  __shared__ __attribute__((aligned(16))) elem sKV[KVLDS ? NWAVES : 1][KVLDS ? NKV : 1][KVLDS ? TILE * D : 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int groups = H / G;
  const BlockXY bxy = work_order_block();
  const int b = bxy.y / groups, gi = bxy.y % groups;
  const int hd0 = gi * G;
  const bool has_h0 = (gi == 0);
  const int NB = (T + TILE - 1) / TILE;
  const int key0 = bxy.x * (NWAVES * TILE) + wave * TILE;
  const int j = key0 + n;
  const int64_t seq_row = (int64_t)b * H;
  // view accessors (CV: the contiguous layout, strides as compile-time facts)
  auto view_head = [&](const elem* base, const Strides& vs_, int hh) -> const elem* {
    if constexpr (CV) return base + (seq_row + hh) * T * D;
    else return base + vs_.at(b, hh);
  };
  auto view_ld = [&](const Strides& vs_) -> int64_t {
    if constexpr (CV) return D;
    else return vs_.row;
  };
  float* uplane = ucheck + ((int64_t)gi * nseq + b) * utri_floats(NB);
  const float* carry_col = carry + (int64_t)b * NB * T + (j < T ? j : 0);

  // Key-side operands (B operands: lane = key column): this wavefront's K and V rows of the group
  // and head 0's K rows, in its LDS rows or in registers.
  frag kf[KVLDS ? 1 : G][NS], vf[KVLDS ? 1 : G][NS], k0f[NS];
  if constexpr (KVLDS) {
    constexpr int CPR = D / 8;
    for (int c = lane; c < TILE * CPR; c += 64) {
      const int r = c / CPR, cc = c % CPR;
      const int64_t jr = min(key0 + r, T - 1);
      const bool ok = key0 + r < T;
      auto put = [&](int x, const elem* src, int64_t ld) {
        const uint4 v4 = *reinterpret_cast<const uint4*>(src + jr * ld + cc * 8);
        *reinterpret_cast<uint4*>(&sKV[wave][x][swz64(r, cc)]) =
            make_uint4(ok ? v4.x : 0u, ok ? v4.y : 0u, ok ? v4.z : 0u, ok ? v4.w : 0u);
      };
#pragma unroll
      for (int g = 0; g < G; ++g) {
        put(2 * g, view_head(k, ks, hd0 + g), view_ld(ks));
        put(2 * g + 1, view_head(v, vs, hd0 + g), view_ld(vs));
      }
    }
    if (!has_h0) {
      const elem* kh = view_head(k, ks, 0);
#pragma unroll
      for (int s = 0; s < NS; ++s) k0f[s] = ld_std_bounded<OP>(kh, view_ld(ks), j, T, h, s);
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const elem* kh = view_head(k, ks, hd0 + g);
      const elem* vh = view_head(v, vs, hd0 + g);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kf[g][s] = ld_std_bounded<OP>(kh, view_ld(ks), j, T, h, s);
        vf[g][s] = ld_std_bounded<OP>(vh, view_ld(vs), j, T, h, s);
      }
    }
    if (!has_h0) {
      const elem* kh = view_head(k, ks, 0);
#pragma unroll
      for (int s = 0; s < NS; ++s) k0f[s] = ld_std_bounded<OP>(kh, view_ld(ks), j, T, h, s);
    }
  }
  // fragment s of row n (this lane's key) of LDS row block x
  auto kv_lds = [&](int x, int s) -> frag {
    if constexpr (KVLDS) return *reinterpret_cast<const frag*>(&sKV[wave][x][swz64(n, 2 * s + h)]);
    else return OP::zero();
  };
  auto k_frag = [&](int g, int s) -> frag {
    if constexpr (KVLDS) return kv_lds(2 * g, s);
    else return kf[g][s];
  };
  auto v_frag = [&](int g, int s) -> frag {
    if constexpr (KVLDS) return kv_lds(2 * g + 1, s);
    else return vf[g][s];
  };
  // head 0's K: the group's own when it holds head 0 (h0)
  auto k0_frag = [&](bool h0, int s) -> frag {
    if constexpr (KVLDS) {
      return h0 ? kv_lds(0, s) : k0f[s];
    } else {
      return h0 ? kf[0][s] : k0f[s];
    }
  };

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
  const float neg_inv_scale = -1.f / scale;
  // query tiles the workgroup visits, last to first: NB-1 down to the first that reaches its keys
  const int qb_lo = bxy.x * NWAVES;
  const int ntiles = NB - qb_lo;

  // Staging of one query tile: Q, Q^T, dO, dO^T of the group (+ head 0's Q, Q^T), lse, dbar.
  RowTile<elem, D> nQ[NH], ndO[G];
  ColTile<elem, D> nQt[NH], ndOt[G];
  float nLse[G], nDb[G];
  // the query-side rows of this workgroup's heads (computed once, outside the tile loop)
  const elem* q_rows[NH];
  const elem* do_rows[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    q_rows[g] = view_head(q, qs, hd0 + g);
    do_rows[g] = view_head(dout, dos, hd0 + g);
  }
  q_rows[G] = view_head(q, qs, 0);
  const int q_ld = (int)view_ld(qs), do_ld = (int)view_ld(dos);
  auto load_tile = [&](int qb) {
    const int qbase = qb * TILE;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t row = seq_row + hd0 + g;
      nQ[g].load(q_rows[g], q_ld, qbase, T, tid);
      nQt[g].load(qt + row * D * ldt, ldt, qbase, tid);
      ndO[g].load(do_rows[g], do_ld, qbase, T, tid);
      ndOt[g].load(dot + row * D * ldt, ldt, qbase, tid);
      const int r = qbase + (tid & (TILE - 1));   // < ldt: padded rows hold lse = +inf, -dbar = 0
      nLse[g] = lse[row * ldt + r];
      nDb[g] = dbar[row * ldt + r];
    }
    if (!has_h0) {
      nQ[G].load(q_rows[G], q_ld, qbase, T, tid);
      nQt[G].load(qt + seq_row * D * ldt, ldt, qbase, tid);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      nQ[g].template store<LDK>(sQ[g], tid);
      nQt[g].template store_crow<LDV>(sQt[g], tid);
      ndO[g].template store<LDK>(sdO[g], tid);
      ndOt[g].template store_crow<LDV>(sdOt[g], tid);
      if (tid < TILE) {
        sLse[g][tid] = nLse[g];
        sDb[g][tid] = nDb[g];
      }
    }
    if (!has_h0) {
      nQ[G].template store<LDK>(sQ[G], tid);
      nQt[G].template store_crow<LDV>(sQt[G], tid);
    }
  };

  // acc[db] (D x keys) += Y^T X: Y a staged transposed LDS tile (rows d, queries in C-layout
  // order), X a C-layout (queries x keys) tile; with split, X also enters as its rounding residual.
  auto acc_t = [&](f32x16 (&acc)[DB], const elem* yt, const f32x16& x, bool split) {
    frag xf[AS];
#pragma unroll
    for (int s = 0; s < AS; ++s) xf[s] = OP::from_acc(x, s);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s) acc[db] = OP::mma(OP::ld_perm(yt, LDV, db * 32 + n, h, s), xf[s], acc[db]);
    if constexpr (OP::SPLIT) {
      if (split) {
#pragma unroll
        for (int s = 0; s < AS; ++s) xf[s] = OP::from_acc_lo(x, s);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int s = 0; s < AS; ++s) acc[db] = OP::mma(OP::ld_perm(yt, LDV, db * 32 + n, h, s), xf[s], acc[db]);
      }
    }
  };

  // Keys below `exempt` are never selected, so they gather attention from every later query and
  // their dV / dK sums run over all of them: their products take the split operands.
  const bool split_keys = key0 < exempt;

  // The tile loop in two instances, for the group holding head 0 and for the others: one loop
  // with a run-time choice between their accumulations makes the compiler copy the sums between
  // register sets every tile.
  auto sweep = [&](auto h0_tag) {
    constexpr bool H0 = decltype(h0_tag)::value;

    // one query tile; INTERIOR: every pair of the tile is unmasked for every wavefront and no key
    // is exempt, so the body is straight-line code without the masks and split products
    auto tile_step = [&](int t, auto interior_tag) {
      constexpr bool INTERIOR = decltype(interior_tag)::value;
      const int qb = NB - 1 - t;
      const int qbase = qb * TILE;
      load_tile(qb);
      const float hist = carry_col[(int64_t)qb * T];
      if (t > 0) __syncthreads();   // every wavefront is done with the previous tile
      store_tile();
      __syncthreads();
      if (INTERIOR || qbase + TILE - 1 >= key0) {   // else every query of the tile precedes every key
        if (h == 0 && j < T) uplane[utri_row(qb) + j] = ucarry;   // j < (qb + 1) * TILE here
        // tile body; edge: some pair of the tile is masked (diagonal, sequence end) or exempt
        // (rows past the end and keys past the end need no mask on the key side: the latter's sums
        // stay in their own lanes, which are never written)
        const bool edge = !INTERIOR && ((qbase <= key0 + TILE - 1) || key0 < exempt);
        const bool split = !INTERIOR && split_keys;
        const TileMasks mk(j, qbase, T, exempt, h);
        // (a lambda: inlined late, its loop-invariant parts are not hoisted out of the tile loop,
        // which would hold them in registers across it)
        auto body = [&]() {
          const elem* q0s = H0 ? sQ[0] : sQ[G];
          f32x16 l0 = zero16();
  #pragma unroll
          for (int s = 0; s < NS; ++s) l0 = OP::mma(OP::ld_std(q0s, LDK, n, h, s), k0_frag(H0, s), l0);
          f32x16 fs;
          uint32_t gate;
          selection_tile<false>(l0, (j < T) ? hist * neg_inv_scale : 0.f, h, edge, mk, gate, fs);

          // Per head: P and dz, dV^T += dO^T P, dK^T += Q^T dz; then g from the group's dz sum goes to
          // head 0's dK: added to head 0's own dz when the group holds it, else into dk0t.
          f32x16 dzsum, dz0;
  #pragma unroll
          for (int g = 0; g < G; ++g) {
            f32x16 lg;   // q.k - F/s
            if (H0 && g == 0) {   // head 0 itself: its logits are l0
  #pragma unroll
              for (int i = 0; i < 16; ++i) lg[i] = l0[i] + fs[i];
            } else {
              lg = fs;
  #pragma unroll
              for (int s = 0; s < NS; ++s) lg = OP::mma(OP::ld_std(sQ[g], LDK, n, h, s), k_frag(g, s), lg);
            }
            f32x16 dp = rows16(sDb[g], h);   // dO.v - dbar
  #pragma unroll
            for (int s = 0; s < NS; ++s) dp = OP::mma(OP::ld_std(sdO[g], LDK, n, h, s), v_frag(g, s), dp);
            f32x16 pr, dz;
            p_dz_tile<false>(lg, dp, sLse[g], sl2, h, edge, mk, pr, dz);
            acc_t(dvt[g], sdOt[g], pr, split);
            if (g == 0) {
              dzsum = dz;
            } else {
  #pragma unroll
              for (int i = 0; i < 16; ++i) dzsum[i] += dz[i];
            }
            if (H0 && g == 0) dz0 = dz;   // head 0's dK waits for g
            else acc_t(dkt[g], sQt[g], dz, split);
          }
          f32x16 gp;
          ucarry = gpath_tile(dzsum, ucarry, gate, h, gp);
          if constexpr (H0) {
  #pragma unroll
            for (int i = 0; i < 16; ++i) dz0[i] += gp[i];
            acc_t(dkt[0], sQt[0], dz0, true);
          } else {
            acc_t(dk0t, sQt[G], gp, big_tile(gp));
          }
        };
        body();
      }
    };
    // The last NWAVES tiles hold the wavefronts' diagonals; a workgroup with an exempt key runs
    // every tile with the masks.
    const int n_int = (qb_lo * TILE < exempt) ? 0 : max(ntiles - NWAVES, 0);
    for (int t = 0; t < n_int; ++t) tile_step(t, std::true_type{});
    for (int t = n_int; t < ntiles; ++t) tile_step(t, std::false_type{});
  };
  if (has_h0) sweep(std::true_type{});
  else sweep(std::false_type{});

  if (j >= T) return;
  // dV of every head and dK of heads other than 0 go to the caller's views; head 0's dK to its
  // fp32 sums, where the other groups' shares join it
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int hh = hd0 + g;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d = db * 32 + 8 * a + 4 * h;
        const float4 kq = make_float4(dkt[g][db][4 * a] * scale, dkt[g][db][4 * a + 1] * scale,
                                      dkt[g][db][4 * a + 2] * scale, dkt[g][db][4 * a + 3] * scale);
        store_grad4(dvv, b, hh, j, d,
                    make_float4(dvt[g][db][4 * a], dvt[g][db][4 * a + 1], dvt[g][db][4 * a + 2], dvt[g][db][4 * a + 3]));
        if (hh == 0 && H > 1) *reinterpret_cast<float4*>(dk0h + ((int64_t)b * T + j) * D + d) = kq;
        else store_grad4(dkv, b, hh, j, d, kq);
      }
  }
  if (!has_h0) {   // this group's share of head 0's dK, in its own slot (group gi: slot gi - 1)
    float* dst = dk0x + ((int64_t)(gi - 1) * nseq * T + (int64_t)b * T + j) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *reinterpret_cast<float4*>(dst + db * 32 + 8 * a + 4 * h) =
            make_float4(dk0t[db][4 * a] * scale, dk0t[db][4 * a + 1] * scale, dk0t[db][4 * a + 2] * scale,
                        dk0t[db][4 * a + 3] * scale);
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, key side, bf16 storage at head dim 64 with one head per wavefront (the instance of
// C2, C3, C4's model and C5): bwd_kv_kernel's tile work, with every query tile's operands loaded
// straight from global memory into LDS one tile ahead -- no staging registers, no load latency at
// the start of a tile, one barrier per tile -- into two buffers of unpadded, swizzled tiles: the Q
// and dO rows (and head 0's Q rows) in swzq layout, read as rows by the logit products and
// transposed (get_trq) by the dK, dV products, so no transposed copies are loaded. The wavefront's
// own K rows sit in registers beside head 0's, its V rows in LDS.

// One tile buffer of bwd_kv64_kernel: the Q, dO and head 0's Q rows (swzq), the rows' lse and
// -dbar (slots 32.. repeat rows 0..31), and per wavefront each lane's carry at the tile's first query.
struct KvTileBuf64 {
  __attribute__((aligned(16))) uint16_t r[3][TILE * 64];
  __attribute__((aligned(16))) float stat[2][64];
  __attribute__((aligned(16))) float hist[NWAVES][64];
};

// CV: every view is the contiguous (nseq, H, T, D) layout of sa_backward. SOLO: one-head sequences
// only (every workgroup runs head 0's loop; the other heads' loop, with its registers for head 0's
// K rows and dK share, is not built).
template <bool CV, bool SOLO>
__global__ __launch_bounds__(NTHREADS, 2) void bwd_kv64_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, Strides qs, Strides ks, Strides vs, Strides dos,
    const float* __restrict__ lse, const float* __restrict__ dbar, const float* __restrict__ carry,
    float* __restrict__ ucheck, float* __restrict__ dk0h, float* __restrict__ dk0x, GradView dkv, GradView dvv,
    int nseq, int H, int T, int64_t ldt, int exempt, float scale) {
  using OP = OpBF16;
  using elem = uint16_t;
  using frag = OP::frag;
  constexpr int D = 64, NS = 4, DB = 2, AS = 2;
  constexpr int TW = TILE * D;   // elements of a [32][64] tile
  // The two tile buffers are separate LDS variables, and the tile loop runs in pairs so that
  // every access names its buffer at compile time: the compiler then knows the direct loads into
  // one buffer do not write what the tile reads from the other, and waits for them only at the end
  // of the tile (a single array indexed by tile parity made it wait before the tile's first read).
  // LDS lifetimes (tile t = query tile NB - 1 - t):
  //   sB0, sB1  tile t's Q, dO and head 0's Q rows, its rows' lse and -dbar, each wavefront's carry
  //             row, buffer t mod 2. Filled: by direct loads of all four wavefronts (rows a quarter
  //             each; statistics by wavefronts 0 and 1; each its own carry row), for tile 0 before
  //             the first barrier, for tile t in tile step t - 1. Drained: tile step t only (every
  //             product's fragment reads, rows16 / p_dz_tile of the statistics, the carry value; a
  //             wavefront with no pair in the tile reads nothing but still loads and synchronises).
  //             Separated: each tile step ends with wait_loads() (this wavefront's loads into the
  //             other buffer have landed) and __syncthreads() (every wavefront's have, and every
  //             wavefront is past its reads of this buffer), so the fill in tile step t + 1 of the
  //             buffer tile step t read follows that barrier, and tile step t + 1's reads of the
  //             buffer filled in tile step t follow it too. The last tile step loads nothing.
  //   sV        per wavefront, its own V rows: written once with plain stores before the first
  //             barrier, only read after it.
  __shared__ KvTileBuf64 sB0, sB1;
  __shared__ __attribute__((aligned(16))) elem sV[NWAVES][TW];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const BlockXY bxy = work_order_block();
  const int b = bxy.y / H, hh = bxy.y % H;
  const bool has_h0 = (hh == 0);
  const int NB = (T + TILE - 1) / TILE;
  const int key0 = bxy.x * (NWAVES * TILE) + wave * TILE;
  const int j = key0 + n;
  const int64_t seq_row = (int64_t)b * H;
  auto view_head = [&](const elem* base, const Strides& s_, int hd) -> const elem* {
    if constexpr (CV) return base + (seq_row + hd) * T * D;
    else return base + s_.at(b, hd);
  };
  auto view_ld = [&](const Strides& s_) -> int {
    if constexpr (CV) return D;
    else return (int)s_.row;
  };
  float* uplane = ucheck + ((int64_t)hh * nseq + b) * utri_floats(NB);
  const float* carry_b = carry + (int64_t)b * NB * T;

  // B operands (lane = key): the wavefront's K rows and head 0's in registers, its V rows in LDS
  frag kf[NS], k0f[NS];
  {
    const elem* kh = view_head(k, ks, hh);
    const elem* k0 = view_head(k, ks, 0);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      kf[s] = ld_std_bounded<OP>(kh, view_ld(ks), j, T, h, s);
      k0f[s] = has_h0 ? kf[s] : ld_std_bounded<OP>(k0, view_ld(ks), j, T, h, s);
    }
    const elem* vh = view_head(v, vs, hh);
    for (int c = lane; c < TILE * (D / 8); c += 64) {
      const int r = c / (D / 8), cc = c % (D / 8);
      const bool ok = key0 + r < T;
      const uint4 v4 = *reinterpret_cast<const uint4*>(vh + (int64_t)(ok ? key0 + r : 0) * view_ld(vs) + cc * 8);
      *reinterpret_cast<uint4*>(&sV[wave][swzq(r, cc)]) = ok ? v4 : make_uint4(0u, 0u, 0u, 0u);
    }
  }

  f32x16 dkt[DB], dvt[DB], dk0t[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dkt[db] = zero16();
    dvt[db] = zero16();
    dk0t[db] = zero16();
  }
  float ucarry = 0.f;
  const float sl2 = scale * LOG2E;
  const float neg_inv_scale = -1.f / scale;
  // query tiles the workgroup visits, last to first: NB-1 down to the first that reaches its keys
  const int qb_lo = bxy.x * NWAVES;
  const int ntiles = NB - qb_lo;

  // operand sources (buffer resources over one head's rows) and this lane's parts of the direct
  // loads
  const int q_ld = view_ld(qs), do_ld = view_ld(dos);
  const __amdgpu_buffer_rsrc_t rs_q = rsrc(view_head(q, qs, hh), (int64_t)T * q_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_do = rsrc(view_head(dout, dos, hh), (int64_t)T * do_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_q0 = rsrc(view_head(q, qs, 0), (int64_t)T * q_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_lse = rsrc(lse + (seq_row + hh) * ldt, ldt * 4);
  const __amdgpu_buffer_rsrc_t rs_ndb = rsrc(dbar + (seq_row + hh) * ldt, ldt * 4);
  const RowsLaneQ rl_q(q_ld, lane, wave), rl_do(do_ld, lane, wave);

  // Everything query tile qb needs, into buffer B, by direct loads only (the tile loop holds no
  // register loads: the vector-memory counter drains in issue order, so waiting for one would wait
  // for the tiles behind it): part `wave` of each operand tile (each wavefront loads a quarter of
  // every tile), the row statistics (wavefronts 0, 1), and each wavefront's carry row of its keys
  // (keys past the end read zero). Tiles load in order, last to first, so the carry row steps back
  // one row per call.
  const float* carry_row = carry_b + (int64_t)(NB - 1) * T;
  auto load_tile = [&](int qb, KvTileBuf64& B) {
    const int qbase = qb * TILE;
    if (wave == 0)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_lse, lds_ptr(B.stat[0]), 4, (lane & 31) * 4, qbase * 4, 0, 0);
    if (wave == 1)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_ndb, lds_ptr(B.stat[1]), 4, (lane & 31) * 4, qbase * 4, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(carry_row, (int64_t)T * 4), lds_ptr(B.hist[wave]), 4, j * 4, 0, 0,
                                             0);
    carry_row -= T;
    g2l_rowsq(B.r[0], rs_q, rl_q, q_ld, qbase, wave);
    g2l_rowsq(B.r[1], rs_do, rl_do, do_ld, qbase, wave);
    if (!has_h0) g2l_rowsq(B.r[2], rs_q0, rl_q, q_ld, qbase, wave);
  };
  // the first tile (NB - 1)
  load_tile(NB - 1, sB0);
  wait_loads();
  __syncthreads();

  // acc[db] (D x keys) += Y^T X: Y a (queries x D) row tile (swzq, read transposed), X a C-layout
  // (queries x keys) tile; with split, X also enters as its rounding residual.
  auto acc_t = [&](f32x16 (&acc)[DB], const elem* y, const f32x16& x, bool split) {
    frag xf[AS];
#pragma unroll
    for (int s = 0; s < AS; ++s) xf[s] = OP::from_acc(x, s);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s) acc[db] = OP::mma(get_trq<true>(y, lane, db, s), xf[s], acc[db]);
    if (split) {
#pragma unroll
      for (int s = 0; s < AS; ++s) xf[s] = OP::from_acc_lo(x, s);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int s = 0; s < AS; ++s) acc[db] = OP::mma(get_trq<true>(y, lane, db, s), xf[s], acc[db]);
    }
  };
  // fragment s of row n of a swzq tile (A operand: lane = query row; or B: lane = key)
  auto rfrag = [&](const elem* tile, int s) -> frag {
    return *reinterpret_cast<const frag*>(tile + swzq(n, 2 * s + h));
  };

  // Keys below `exempt` are never selected, so they gather attention from every later query and
  // their dV / dK sums run over all of them: their products take the split operands.
  const bool split_keys = key0 < exempt;

  // the tile loop in two instances, for head 0's workgroups and the others (see bwd_kv_kernel)
  auto sweep = [&](auto h0_tag) {
    constexpr bool H0 = decltype(h0_tag)::value;
    // the checkpoint row of tile t's query block (the rows lie end to end, tiles run last to first)
    float* urow = uplane + utri_row(NB - 1);
    // tile t (buffer t mod 2, named by ODD)
    auto tile_step = [&](int t, auto interior_tag, auto odd_tag) {
      constexpr bool INTERIOR = decltype(interior_tag)::value;
      constexpr bool ODD = decltype(odd_tag)::value;
      KvTileBuf64& B = ODD ? sB1 : sB0;
      const int qb = NB - 1 - t;
      const int qbase = qb * TILE;
      const bool more = t + 1 < ntiles;
      if (more) load_tile(qb - 1, ODD ? sB0 : sB1);   // into the other buffer, free since the last barrier
      if (INTERIOR || qbase + TILE - 1 >= key0) {   // else every query of the tile precedes every key
        if (h == 0 && j < T) urow[j] = ucarry;   // j < (qb + 1) * TILE here
        const bool edge = !INTERIOR && ((qbase <= key0 + TILE - 1) || key0 < exempt);
        const bool split = !INTERIOR && split_keys;
        const TileMasks mk(j, qbase, T, exempt, h);
        auto body = [&]() {
          // (keys past the end read a zero carry through the load's range check)
          const float hist = B.hist[wave][lane];
          const elem* q0s = H0 ? B.r[0] : B.r[2];
          // the four fragments of head 0's Q rows are all requested before the chain of logit
          // products starts, so the chain waits for one LDS latency rather than one per product
          // (the default scheduler otherwise issues each read just before its product)
          frag q0r[NS];
#pragma unroll
          for (int s = 0; s < NS; ++s) q0r[s] = rfrag(q0s, s);
          __builtin_amdgcn_sched_barrier(0);
          f32x16 l0 = zero16();
#pragma unroll
          for (int s = 0; s < NS; ++s) l0 = OP::mma(q0r[s], H0 ? kf[s] : k0f[s], l0);
          f32x16 fs;
          uint32_t gate;
          selection_tile<false>(l0, hist * neg_inv_scale, h, edge, mk, gate, fs);

          f32x16 lg;   // q.k - F/s
          if constexpr (H0) {   // head 0 itself: its logits are l0
#pragma unroll
            for (int i = 0; i < 16; ++i) lg[i] = l0[i] + fs[i];
          } else {
            lg = fs;
#pragma unroll
            for (int s = 0; s < NS; ++s) lg = OP::mma(rfrag(B.r[0], s), kf[s], lg);
          }
          f32x16 dp = rows16(B.stat[1], h);   // dO.v - dbar
#pragma unroll
          for (int s = 0; s < NS; ++s) dp = OP::mma(rfrag(B.r[1], s), rfrag(sV[wave], s), dp);
          f32x16 pr, dz;
          p_dz_tile<false>(lg, dp, B.stat[0], sl2, h, edge, mk, pr, dz);
          acc_t(dvt, B.r[1], pr, split);
          f32x16 gp;
          ucarry = gpath_tile(dz, ucarry, gate, h, gp);
          if constexpr (H0) {   // head 0's dK takes g with its own dz
#pragma unroll
            for (int i = 0; i < 16; ++i) dz[i] += gp[i];
            acc_t(dkt, B.r[0], dz, split || big_tile(dz));
          } else {
            acc_t(dkt, B.r[0], dz, split);
            acc_t(dk0t, B.r[2], gp, big_tile(gp));
          }
        };
        body();
      }
      urow -= 32 * qb;   // utri_row(qb - 1)
      wait_loads();
      __syncthreads();   // the next tile's operands are in; every wavefront is done with this one
    };
    // The last NWAVES tiles hold the wavefronts' diagonals; a workgroup with an exempt key runs
    // every tile with the masks.
    const int n_int = (qb_lo * TILE < exempt) ? 0 : max(ntiles - NWAVES, 0);
    // tiles [t0, t1) in pairs, even tiles from buffer 0 and odd ones from buffer 1
    auto run = [&](int t0, int t1, auto interior_tag) {
      int t = t0;
      if (t < t1 && (t & 1)) tile_step(t++, interior_tag, std::true_type{});
      for (; t + 1 < t1; t += 2) {
        tile_step(t, interior_tag, std::false_type{});
        tile_step(t + 1, interior_tag, std::true_type{});
      }
      if (t < t1) tile_step(t, interior_tag, std::false_type{});
    };
    run(0, n_int, std::true_type{});
    run(n_int, ntiles, std::false_type{});
  };
  if (SOLO || has_h0) sweep(std::true_type{});
  else if constexpr (!SOLO) sweep(std::false_type{});

  if (j >= T) return;
  // dV and the dK of heads other than 0 go to the caller's views; head 0's dK to its fp32 sums,
  // where the other heads' shares join it (to its view too when it is the sequence's only head)
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int d = db * 32 + 8 * a + 4 * h;
      const float4 kq = make_float4(dkt[db][4 * a] * scale, dkt[db][4 * a + 1] * scale, dkt[db][4 * a + 2] * scale,
                                    dkt[db][4 * a + 3] * scale);
      store_grad4(dvv, b, hh, j, d, make_float4(dvt[db][4 * a], dvt[db][4 * a + 1], dvt[db][4 * a + 2], dvt[db][4 * a + 3]));
      if (has_h0 && H > 1) *reinterpret_cast<float4*>(dk0h + ((int64_t)b * T + j) * D + d) = kq;
      else store_grad4(dkv, b, hh, j, d, kq);
    }
  if (!has_h0) {   // this head's share of head 0's dK, in its own slot (head hh: slot hh - 1)
    float* dst = dk0x + ((int64_t)(hh - 1) * nseq * T + (int64_t)b * T + j) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int a = 0; a < 4; ++a)
        *reinterpret_cast<float4*>(dst + db * 32 + 8 * a + 4 * h) =
            make_float4(dk0t[db][4 * a] * scale, dk0t[db][4 * a + 1] * scale, dk0t[db][4 * a + 2] * scale,
                        dk0t[db][4 * a + 3] * scale);
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, query side. grid (ceil(T/128), nseq * H/G); wavefront w owns queries
// [x*128 + 32w, +32) of heads [gi*G, gi*G+G) (late query blocks launch first) and walks the key
// tiles up to its diagonal, with Q, dO and the dQ sums in registers. It recomputes P and dz as the
// key side does, and this group's share of head 0's g from the key side's checkpoint of U plus
// the suffix inside the tile. dQ = dz K takes dz through a per-wavefront LDS tile (as the A operand)
// and K^T from LDS (as the B operand).

template <class OP, int D, int G, bool CV>   // CV: see bwd_kv_kernel
__global__ __launch_bounds__(NTHREADS, (dq_min_blocks<OP, D>())) void bwd_dq_kernel(
    const typename OP::elem* __restrict__ q, const typename OP::elem* __restrict__ k,
    const typename OP::elem* __restrict__ v, const typename OP::elem* __restrict__ kt,
    const typename OP::elem* __restrict__ dout, Strides qs, Strides ks, Strides vs, Strides dos,
    const float* __restrict__ lse, const float* __restrict__ dbar, const float* __restrict__ carry,
    const float* __restrict__ ucheck, float* __restrict__ dq0h, float* __restrict__ dq0x, GradView dqv, int nseq,
    int H, int T, int64_t ldt, int exempt, float scale) {
  using elem = typename OP::elem;
  using frag = typename OP::frag;
  constexpr int NS = D / OP::KS;
  constexpr int DB = D / 32;
  constexpr int LDK = D + OP::KPAD;
  constexpr int LDKT = TILE + OP::KPAD;
  constexpr int LDZ = TILE + OP::KPAD;
  constexpr int AS = OP::acc_steps;
  constexpr int NH = G + 1;

  __shared__ __attribute__((aligned(16))) elem sK[NH][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sKt[NH][D * LDKT];
  __shared__ __attribute__((aligned(16))) elem sV[G][TILE * LDK];
  __shared__ __attribute__((aligned(16))) elem sZ[NWAVES][TILE * LDZ];

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const int groups = H / G;
  const BlockXY bxy = work_order_block();
  const int b = bxy.y / groups, gi = bxy.y % groups;
  const int hd0 = gi * G;
  const bool has_h0 = (gi == 0);
  const int NB = (T + TILE - 1) / TILE;
  const int qsb = gridDim.x - 1 - bxy.x;
  const int qb = qsb * NWAVES + wave;
  const int qbase = qb * TILE;
  const int64_t seq_row = (int64_t)b * H;
  // view accessors (CV: the contiguous layout, strides as compile-time facts)
  auto view_head = [&](const elem* base, const Strides& vs_, int hh) -> const elem* {
    if constexpr (CV) return base + (seq_row + hh) * T * D;
    else return base + vs_.at(b, hh);
  };
  auto view_ld = [&](const Strides& vs_) -> int64_t {
    if constexpr (CV) return D;
    else return vs_.row;
  };
  const int my_end = (qb < NB) ? qb + 1 : 0;
  const int wg_end = min(qsb * NWAVES + NWAVES - 1, NB - 1) + 1;
  elem* zs = sZ[wave];
  // this wavefront's rows of the carry and U checkpoints (key offset added per tile)
  const int qb_c = qb < NB ? qb : NB - 1;
  const float* carry_row = carry + ((int64_t)b * NB + qb_c) * T;
  // (the row's keys end at (qb_c + 1) * TILE; the tiles past a wavefront's diagonal read, unused,
  // into the next row, and the last row spans every key tile: the reads stay inside the plane)
  const float* urow = ucheck + ((int64_t)gi * nseq + b) * utri_floats(NB) + utri_row(qb_c);

  // Query-side operands (A operands: lane = query row): the group's Q and dO rows and head 0's Q
  // rows in registers, as are the rows' statistics (element i: row crow(i, h)).
  frag q0a[NS];
  frag qa[G][NS], doa[G][NS];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      qa[g][s] = ld_std_bounded<OP>(view_head(q, qs, hd0 + g), view_ld(qs), qbase + n, T, h, s);
      doa[g][s] = ld_std_bounded<OP>(view_head(dout, dos, hd0 + g), view_ld(dos), qbase + n, T, h, s);
    }
  }
  auto q_frag = [&](int g, int s) -> frag { return qa[g][s]; };
  auto do_frag = [&](int g, int s) -> frag { return doa[g][s]; };
  f32x16 lse_r[G], ndb_r[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t row = seq_row + hd0 + g;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = qbase + crow(i, h);
      const int rr = min(r, T - 1);
      const float lv = lse[row * ldt + rr], dv_ = dbar[row * ldt + rr];
      lse_r[g][i] = (r < T) ? lv : INFINITY;   // rows past the end: P = 0
      ndb_r[g][i] = (r < T) ? dv_ : 0.f;      // -dbar: dO.v accumulates onto it
    }
  }
  if (!has_h0) {
#pragma unroll
    for (int s = 0; s < NS; ++s) q0a[s] = ld_std_bounded<OP>(view_head(q, qs, 0), view_ld(qs), qbase + n, T, h, s);
  }

  f32x16 dqacc[G][DB], dq0acc[DB];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int db = 0; db < DB; ++db) dqacc[g][db] = zero16();
#pragma unroll
  for (int db = 0; db < DB; ++db) dq0acc[db] = zero16();

  const float sl2 = scale * LOG2E;
  const float neg_inv_scale = -1.f / scale;

  // Staging of one key tile: K, V, K^T of the group (+ head 0's K, K^T).
  RowTile<elem, D> nK[NH], nV[G];
  ColTile<elem, D> nKt[NH];
  // the key-side rows of this workgroup's heads (computed once, outside the tile loop)
  const elem* k_rows[NH];
  const elem* v_rows[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    k_rows[g] = view_head(k, ks, hd0 + g);
    v_rows[g] = view_head(v, vs, hd0 + g);
  }
  k_rows[G] = view_head(k, ks, 0);
  const int k_ld = (int)view_ld(ks), v_ld = (int)view_ld(vs);
  auto load_tile = [&](int ktile) {
    const int kbase = ktile * TILE;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t row = seq_row + hd0 + g;
      nK[g].load(k_rows[g], k_ld, kbase, T, tid);
      nV[g].load(v_rows[g], v_ld, kbase, T, tid);
      nKt[g].load(kt + row * D * ldt, ldt, kbase, tid);
    }
    if (!has_h0) {
      nK[G].load(k_rows[G], k_ld, kbase, T, tid);
      nKt[G].load(kt + seq_row * D * ldt, ldt, kbase, tid);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      nK[g].template store<LDK>(sK[g], tid);
      nV[g].template store<LDK>(sV[g], tid);
      nKt[g].template store<LDKT>(sKt[g], tid);
    }
    if (!has_h0) {
      nK[G].template store<LDK>(sK[G], tid);
      nKt[G].template store<LDKT>(sKt[G], tid);
    }
  };

  // acc[db] (queries x D) += X K: X a C-layout (queries x keys) tile, sent through LDS to become
  // the A operand; K^T (rows d) staged in LDS is the B operand. With split, X's rounding residual
  // takes a second pass.
  auto acc_xk = [&](f32x16 (&acc)[DB], const f32x16& x, const elem* ktile, bool split) {
    frag zf[AS];
    if constexpr (sizeof(elem) == 2) {
      // bf16: X goes to the tile transposed (4 rows per write) and comes back through the
      // transposing read
      put_tr<false>(zs, x, n, h);
      lds_wave_sync();
#pragma unroll
      for (int s = 0; s < AS; ++s) zf[s] = get_tr(zs, lane, s);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int s = 0; s < AS; ++s) acc[db] = OP::mma(zf[s], OP::ld_std(ktile, LDKT, db * 32 + n, h, s), acc[db]);
      if (split) {
        lds_wave_sync();
        put_tr<true>(zs, x, n, h);
        lds_wave_sync();
#pragma unroll
        for (int s = 0; s < AS; ++s) zf[s] = get_tr(zs, lane, s);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int s = 0; s < AS; ++s) acc[db] = OP::mma(zf[s], OP::ld_std(ktile, LDKT, db * 32 + n, h, s), acc[db]);
      }
      lds_wave_sync();
      return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) zs[crow(i, h) * LDZ + n] = OP::to_elem(x[i]);
    lds_wave_sync();
#pragma unroll
    for (int s = 0; s < AS; ++s) zf[s] = OP::ld_std(zs, LDZ, n, h, s);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s) acc[db] = OP::mma(zf[s], OP::ld_std(ktile, LDKT, db * 32 + n, h, s), acc[db]);
    if constexpr (OP::SPLIT) {
      if (split) {
        lds_wave_sync();
#pragma unroll
        for (int i = 0; i < 16; ++i) zs[crow(i, h) * LDZ + n] = OP::to_elem_lo(x[i]);
        lds_wave_sync();
#pragma unroll
        for (int s = 0; s < AS; ++s) zf[s] = OP::ld_std(zs, LDZ, n, h, s);
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int s = 0; s < AS; ++s) acc[db] = OP::mma(zf[s], OP::ld_std(ktile, LDKT, db * 32 + n, h, s), acc[db]);
      }
    }
    lds_wave_sync();
  };

  auto key_vals = [&](int ktile, float& hv, float& uv) {
    const int jj = ktile * TILE + n;
    hv = (jj < T) ? carry_row[jj] : 0.f;
    uv = (jj < T) ? urow[jj] : 0.f;
  };

  // The tile loop in two instances, for the group holding head 0 and for the others (as on the
  // key side).
  auto sweep = [&](auto h0_tag) {
    constexpr bool H0 = decltype(h0_tag)::value;

    // one key tile; INTERIOR: no pair of the tile is masked or exempt for any wavefront, so the
    // body is straight-line code without the masks
    auto tile_step = [&](int ktile, auto interior_tag) {
      constexpr bool INTERIOR = decltype(interior_tag)::value;
      const int kbase = ktile * TILE;
      float hist, uin;
      load_tile(ktile);
      key_vals(ktile, hist, uin);
      if (ktile > 0) __syncthreads();   // every wavefront is done with the previous tile
      store_tile();
      __syncthreads();
      if (ktile < my_end) {
        const int j = kbase + n;
        // tile body; edge: some pair of the tile is masked (diagonal, sequence end) or exempt
        const bool edge = !INTERIOR && ((kbase + TILE - 1 >= qbase) || (kbase + TILE > T) || kbase < exempt);
        const TileMasks mk(j, qbase, T, exempt, h);
        {
          const elem* k0s = H0 ? sK[0] : sK[G];
          f32x16 l0 = zero16();
  #pragma unroll
          for (int s = 0; s < NS; ++s)
            l0 = OP::mma(H0 ? q_frag(0, s) : q0a[s], OP::ld_std(k0s, LDK, n, h, s), l0);
          f32x16 fs;
          uint32_t gate;
          selection_tile<false>(l0, hist * neg_inv_scale, h, edge, mk, gate, fs);

          f32x16 zsum, dz0;
  #pragma unroll
          for (int g = 0; g < G; ++g) {
            f32x16 lg;   // q.k - F/s
            if (H0 && g == 0) {   // head 0 itself: its logits are l0, its dQ waits for g
  #pragma unroll
              for (int i = 0; i < 16; ++i) lg[i] = l0[i] + fs[i];
            } else {
              lg = fs;
  #pragma unroll
              for (int s = 0; s < NS; ++s)
                lg = OP::mma(q_frag(g, s), OP::ld_std(sK[g], LDK, n, h, s), lg);
            }
            f32x16 dp;   // dO.v - dbar
            dp = ndb_r[g];
  #pragma unroll
            for (int s = 0; s < NS; ++s)
              dp = OP::mma(do_frag(g, s), OP::ld_std(sV[g], LDK, n, h, s), dp);
            f32x16 pr, dz;
            p_dz_tile_r(lg, dp, lse_r[g], sl2, edge, mk, pr, dz);
            if (g == 0) {
              zsum = dz;
            } else {
  #pragma unroll
              for (int i = 0; i < 16; ++i) zsum[i] += dz[i];
            }
            if (H0 && g == 0) {
              dz0 = dz;
            } else {
              acc_xk(dqacc[g], dz, sKt[g], false);
            }
          }

          f32x16 gp;
          gpath_tile(zsum, uin, gate, h, gp);
          if constexpr (H0) {
            f32x16 dzh;
  #pragma unroll
            for (int i = 0; i < 16; ++i) dzh[i] = dz0[i] + gp[i];
            acc_xk(dqacc[0], dzh, sKt[0], big_tile(dzh));
          } else {
            acc_xk(dq0acc, gp, sKt[G], big_tile(gp));
          }
        }
      }
    };
    // tiles holding exempt keys, then the interior ones (below every wavefront's diagonal, which
    // also keeps them clear of the sequence end), then the diagonals
    const int i_lo = min((exempt + TILE - 1) / TILE, wg_end);
    const int i_hi = max(i_lo, min(qsb * NWAVES, wg_end));
    for (int ktile = 0; ktile < i_lo; ++ktile) tile_step(ktile, std::false_type{});
    for (int ktile = i_lo; ktile < i_hi; ++ktile) tile_step(ktile, std::true_type{});
    for (int ktile = i_hi; ktile < wg_end; ++ktile) tile_step(ktile, std::false_type{});
  };
  if (has_h0) sweep(std::true_type{});
  else sweep(std::false_type{});

  if (qb >= NB) return;
  // heads other than 0: dQ (scaled) to the caller's view; head 0: unscaled fp32 sums, where the
  // other groups' shares join it
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int hh = hd0 + g;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = qbase + crow(i, h);
      if (r < T) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          if (hh == 0 && H > 1) dq0h[((int64_t)b * T + r) * D + db * 32 + n] = dqacc[g][db][i];
          else store_grad1(dqv, b, hh, r, db * 32 + n, dqacc[g][db][i] * scale);
        }
      }
    }
  }
  if (!has_h0) {   // this group's share of head 0's dQ (unscaled), in its own slot (group gi: slot gi - 1)
    float* dst = dq0x + ((int64_t)(gi - 1) * nseq * T + (int64_t)b * T) * D;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = qbase + crow(i, h);
      if (r < T) {
#pragma unroll
        for (int db = 0; db < DB; ++db) dst[(int64_t)r * D + db * 32 + n] = dq0acc[db][i];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, query side, bf16 storage at head dim 64 with one head per wavefront: bwd_dq_kernel's
// tile work with every key tile's operands -- the K, V and head 0's K rows (swzq; the K rows read
// as rows by the logit products and transposed by the dQ products, so no K^T is loaded), and each
// wavefront's carry and selection-suffix checkpoint values of the tile's keys -- loaded straight
// into LDS one tile ahead, two buffers as separate LDS variables (see bwd_kv64_kernel); one barrier
// per tile. Eight wavefronts (256 queries) per workgroup, one
// workgroup per CU: each key tile is staged once for twice the queries of a four-wavefront group
// (measured 3% faster; the operand staging, not its latency, is what the loads cost).

constexpr int DQ64_WAVES = 8;

struct DqTileBuf64 {
  __attribute__((aligned(16))) uint16_t k[2][TILE * 64];    // K rows, head 0's K rows (swzq)
  __attribute__((aligned(16))) uint16_t v[TILE * 64];       // V rows (swzq)
  __attribute__((aligned(16))) float hist[DQ64_WAVES][64];   // per wavefront: each lane's key's carry
  __attribute__((aligned(16))) float uin[DQ64_WAVES][64];    // ... and its U checkpoint
};

// CV: every view is the contiguous (nseq, H, T, D) layout of sa_backward. SOLO: one-head sequences
// only (head 0's loop alone is built, as in bwd_kv64_kernel). SNAKE: workgroups dealt in the order
// of work_order_block(order_slots) (an instance of its own, so the launches in the longest-first
// order run exactly the code they ran before it existed; order_slots is unused there).
template <bool CV, bool SOLO, bool SNAKE = false>
__global__ __launch_bounds__(DQ64_WAVES * 64, 1) void bwd_dq64_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, Strides qs, Strides ks, Strides vs, Strides dos,
    const float* __restrict__ lse, const float* __restrict__ dbar, const float* __restrict__ carry,
    const float* __restrict__ ucheck, float* __restrict__ dq0h, float* __restrict__ dq0x, GradView dqv, int nseq,
    int H, int T, int64_t ldt, int exempt, float scale, int order_slots) {
  using OP = OpBF16;
  using elem = uint16_t;
  using frag = OP::frag;
  constexpr int D = 64, NS = 4, DB = 2, AS = 2;
  // LDS lifetimes (key tile t):
  //   sB0, sB1  tile t's K, head 0's K and V rows, each wavefront's carry and U-checkpoint values,
  //             buffer t mod 2. Filled: by direct loads (K rows by wavefronts 0-3, V rows by 4-7, a
  //             quarter each; every wavefront its own carry and checkpoint values), tile 0 before the
  //             first barrier, tile t in tile step t - 1. Drained: tile step t only (a wavefront
  //             whose diagonal lies before tile t reads nothing but still loads and synchronises).
  //             Separated: as in bwd_kv64_kernel, each tile step ends with wait_loads() and
  //             __syncthreads(), between the last reads of a buffer and its next fill, and between a
  //             fill and its reads. The last tile step loads nothing.
  //   sZ        per wavefront, the dz / g tile transposed for the dQ products: written and read by
  //             the same wavefront within a product (acc_xk); the LDS performs one wavefront's
  //             operations in issue order, so lds_wave_order (a compiler barrier) keeps each read
  //             after its write and the next write after the reads.
  //   sRow      per wavefront, its rows' lse and -dbar: written once before the first barrier, only
  //             read after it.
  __shared__ DqTileBuf64 sB0, sB1;
  __shared__ __attribute__((aligned(16))) elem sZ[DQ64_WAVES][TILE * TILE];   // per wavefront: dz, g transposed
  __shared__ __attribute__((aligned(16))) float sRow[DQ64_WAVES][2][TILE];   // per wavefront: its rows' lse, -dbar

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int n = lane & 31, h = lane >> 5;
  const BlockXY bxy = SNAKE ? work_order_block(order_slots) : work_order_block();
  const int b = bxy.y / H, hh = bxy.y % H;
  const bool has_h0 = (hh == 0);
  const int NB = (T + TILE - 1) / TILE;
  const int qsb = gridDim.x - 1 - bxy.x;
  const int qb = qsb * DQ64_WAVES + wave;
  const int qbase = qb * TILE;
  const int64_t seq_row = (int64_t)b * H;
  auto view_head = [&](const elem* base, const Strides& s_, int hd) -> const elem* {
    if constexpr (CV) return base + (seq_row + hd) * T * D;
    else return base + s_.at(b, hd);
  };
  auto view_ld = [&](const Strides& s_) -> int {
    if constexpr (CV) return D;
    else return (int)s_.row;
  };
  const int my_end = (qb < NB) ? qb + 1 : 0;
  const int wg_end = min(qsb * DQ64_WAVES + DQ64_WAVES - 1, NB - 1) + 1;
  elem* zs = sZ[wave];
  const int qb_c = qb < NB ? qb : NB - 1;

  // A operands (lane = query row): the Q, dO rows and head 0's Q rows in registers; the rows'
  // statistics in the wavefront's LDS rows (registers would spill)
  frag qa[NS], doa[NS], q0a[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qa[s] = ld_std_bounded<OP>(view_head(q, qs, hh), view_ld(qs), qbase + n, T, h, s);
    doa[s] = ld_std_bounded<OP>(view_head(dout, dos, hh), view_ld(dos), qbase + n, T, h, s);
  }
  if (!has_h0) {
#pragma unroll
    for (int s = 0; s < NS; ++s) q0a[s] = ld_std_bounded<OP>(view_head(q, qs, 0), view_ld(qs), qbase + n, T, h, s);
  }
  if (lane < TILE) {
    const int64_t row = seq_row + hh;
    const int r = qbase + lane;
    const int rr = min(r, T - 1);
    const float lv = lse[row * ldt + rr], dv_ = dbar[row * ldt + rr];
    sRow[wave][0][lane] = (r < T) ? lv : INFINITY;   // rows past the end: P = 0
    sRow[wave][1][lane] = (r < T) ? dv_ : 0.f;       // -dbar: dO.v accumulates onto it
  }

  f32x16 dqacc[DB], dq0acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dqacc[db] = zero16();
    dq0acc[db] = zero16();
  }
  const float sl2 = scale * LOG2E;
  const float neg_inv_scale = -1.f / scale;

  // key-side sources (buffer resources over one head's rows), this wavefront's rows of the carry
  // and of the U checkpoints (keys past them read zero)
  const int k_ld = view_ld(ks), v_ld = view_ld(vs);
  const __amdgpu_buffer_rsrc_t rs_k = rsrc(view_head(k, ks, hh), (int64_t)T * k_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_k0 = rsrc(view_head(k, ks, 0), (int64_t)T * k_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_v = rsrc(view_head(v, vs, hh), (int64_t)T * v_ld * 2);
  const __amdgpu_buffer_rsrc_t rs_c = rsrc(carry + ((int64_t)b * NB + qb_c) * T, (int64_t)T * 4);
  const __amdgpu_buffer_rsrc_t rs_u =
      rsrc(ucheck + ((int64_t)hh * nseq + b) * utri_floats(NB) + utri_row(qb_c), (int64_t)(qb_c + 1) * TILE * 4);
  const RowsLaneQ rl_k(k_ld, lane, wave & 3), rl_v(v_ld, lane, wave & 3);

  // everything key tile ktile needs, into buffer B, by direct loads only (see bwd_kv64_kernel):
  // wavefronts 0-3 load a quarter of the K rows (and of head 0's), 4-7 of the V rows
  auto load_tile = [&](int ktile, DqTileBuf64& B) {
    const int kbase = ktile * TILE;
    const int m = wave & 3;
    if (wave < 4) {
      g2l_rowsq(B.k[0], rs_k, rl_k, k_ld, kbase, m);
      if (!has_h0) g2l_rowsq(B.k[1], rs_k0, rl_k, k_ld, kbase, m);
    } else {
      g2l_rowsq(B.v, rs_v, rl_v, v_ld, kbase, m);
    }
    const int jo = (kbase + n) * 4;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_c, lds_ptr(B.hist[wave]), 4, jo, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_u, lds_ptr(B.uin[wave]), 4, jo, 0, 0, 0);
  };
  // fragment s of row n (lane = key) of a swzq tile
  auto rfrag = [&](const elem* tile, int s) -> frag {
    return *reinterpret_cast<const frag*>(tile + swzq(n, 2 * s + h));
  };
  // acc[db] (queries x D) += X K: X a C-layout (queries x keys) tile sent through the wavefront's
  // LDS tile to become the A operand (transposed write, transposing read), the K rows (swzq) read
  // transposed as the B operand; with split, X's rounding residual takes a second pass.
  // The tile zs is the wavefront's own: its writes and reads are ordered by lds_wave_order (the
  // previous tile's reads of zs precede this tile's writes in program order as well).
  auto acc_xk = [&](f32x16 (&acc)[DB], const f32x16& x, const elem* ktile, bool split) {
    frag zf[AS];
    put_tr<false>(zs, x, n, h);
    lds_wave_order();
#pragma unroll
    for (int s = 0; s < AS; ++s) zf[s] = get_tr(zs, lane, s);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int s = 0; s < AS; ++s)
        acc[db] = OP::mma(zf[s], get_trq<false>(ktile, lane, db, s), acc[db]);
    if (split) {
      lds_wave_order();
      put_tr<true>(zs, x, n, h);
      lds_wave_order();
#pragma unroll
      for (int s = 0; s < AS; ++s) zf[s] = get_tr(zs, lane, s);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int s = 0; s < AS; ++s)
          acc[db] = OP::mma(zf[s], get_trq<false>(ktile, lane, db, s), acc[db]);
    }
    lds_wave_order();
  };

  // the first key tile
  load_tile(0, sB0);
  wait_loads();
  __syncthreads();

  // the tile loop in two instances, for head 0's workgroups and the others (see bwd_kv_kernel)
  auto sweep = [&](auto h0_tag) {
    constexpr bool H0 = decltype(h0_tag)::value;
    // key tile ktile (buffer ktile mod 2, named by ODD); INTERIOR: no pair of the tile is masked or
    // exempt for any wavefront
    auto tile_step = [&](int ktile, auto interior_tag, auto odd_tag) {
      constexpr bool INTERIOR = decltype(interior_tag)::value;
      constexpr bool ODD = decltype(odd_tag)::value;
      DqTileBuf64& B = ODD ? sB1 : sB0;
      const int kbase = ktile * TILE;
      if (ktile + 1 < wg_end) load_tile(ktile + 1, ODD ? sB0 : sB1);   // free since the last barrier
      if (ktile < my_end) {
        const int j = kbase + n;
        const bool edge = !INTERIOR && ((kbase + TILE - 1 >= qbase) || (kbase + TILE > T) || kbase < exempt);
        const TileMasks mk(j, qbase, T, exempt, h);
        const float hist = B.hist[wave][lane], uin = B.uin[wave][lane];
        const elem* k0s = H0 ? B.k[0] : B.k[1];
        f32x16 l0 = zero16();
#pragma unroll
        for (int s = 0; s < NS; ++s) l0 = OP::mma(H0 ? qa[s] : q0a[s], rfrag(k0s, s), l0);
        f32x16 fs;
        uint32_t gate;
        selection_tile<false>(l0, hist * neg_inv_scale, h, edge, mk, gate, fs);
        f32x16 lg;   // q.k - F/s
        if constexpr (H0) {   // head 0 itself: its logits are l0
#pragma unroll
          for (int i = 0; i < 16; ++i) lg[i] = l0[i] + fs[i];
        } else {
          lg = fs;
#pragma unroll
          for (int s = 0; s < NS; ++s) lg = OP::mma(qa[s], rfrag(B.k[0], s), lg);
        }
        f32x16 dp = rows16(sRow[wave][1], h);   // dO.v - dbar
#pragma unroll
        for (int s = 0; s < NS; ++s) dp = OP::mma(doa[s], rfrag(B.v, s), dp);
        f32x16 pr, dz;
        p_dz_tile<false>(lg, dp, sRow[wave][0], sl2, h, edge, mk, pr, dz);
        f32x16 gp;
        gpath_tile(dz, uin, gate, h, gp);
        if constexpr (H0) {   // head 0's dQ takes g with its own dz
#pragma unroll
          for (int i = 0; i < 16; ++i) dz[i] += gp[i];
          acc_xk(dqacc, dz, B.k[0], big_tile(dz));
        } else {
          acc_xk(dqacc, dz, B.k[0], false);
          acc_xk(dq0acc, gp, B.k[1], big_tile(gp));
        }
      }
      wait_loads();
      __syncthreads();   // the next tile's operands are in; every wavefront is done with this one
    };
    auto run = [&](int t0, int t1, auto interior_tag) {
      int t = t0;
      if (t < t1 && (t & 1)) tile_step(t++, interior_tag, std::true_type{});
      for (; t + 1 < t1; t += 2) {
        tile_step(t, interior_tag, std::false_type{});
        tile_step(t + 1, interior_tag, std::true_type{});
      }
      if (t < t1) tile_step(t, interior_tag, std::false_type{});
    };
    // tiles holding exempt keys, then the interior ones (below every wavefront's diagonal, which
    // also keeps them clear of the sequence end), then the diagonals
    const int i_lo = min((exempt + TILE - 1) / TILE, wg_end);
    const int i_hi = max(i_lo, min(qsb * DQ64_WAVES, wg_end));
    run(0, i_lo, std::false_type{});
    run(i_lo, i_hi, std::true_type{});
    run(i_hi, wg_end, std::false_type{});
  };
  if (SOLO || has_h0) sweep(std::true_type{});
  else if constexpr (!SOLO) sweep(std::false_type{});

  if (qb >= NB) return;
  // heads other than 0: dQ (scaled) to the caller's view; head 0: unscaled fp32 sums, where the
  // other heads' shares join it (to its view too when it is the sequence's only head)
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = qbase + crow(i, h);
    if (r < T) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        if (has_h0 && H > 1) dq0h[((int64_t)b * T + r) * D + db * 32 + n] = dqacc[db][i];
        else store_grad1(dqv, b, hh, r, db * 32 + n, dqacc[db][i] * scale);
      }
    }
  }
  if (!has_h0) {   // this head's share of head 0's dQ (unscaled), in its own slot (head hh: slot hh - 1)
    float* dst = dq0x + ((int64_t)(hh - 1) * nseq * T + (int64_t)b * T) * D;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = qbase + crow(i, h);
      if (r < T) {
#pragma unroll
        for (int db = 0; db < DB; ++db) dst[(int64_t)r * D + db * 32 + n] = dq0acc[db][i];
      }
    }
  }
}

// Head 0's gradients: its own fp32 sums plus the other groups' shares, summed slot after slot in
// group order (so every run adds the same values in the same order), (b, t, D) contiguous, four
// elements per thread, to the caller's views. nslots slots of total4 float4s each.
__global__ __launch_bounds__(NTHREADS) void bwd_finish_kernel(
    const float4* __restrict__ dq0h, const float4* __restrict__ dk0h, const float4* __restrict__ dq0x,
    const float4* __restrict__ dk0x, int nslots, GradView dqv, GradView dkv, int D, int64_t TD, int64_t total4,
    float scale) {
  for (int64_t e = (int64_t)blockIdx.x * NTHREADS + threadIdx.x; e < total4; e += (int64_t)gridDim.x * NTHREADS) {
    const int64_t b = (4 * e) / TD, off = 4 * e - b * TD;
    const int t = (int)(off / D), d = (int)(off - (int64_t)t * D);
    float4 q = dq0h[e], k = dk0h[e];
    for (int sl = 0; sl < nslots; ++sl) {
      const float4 qx = dq0x[sl * total4 + e], kx = dk0x[sl * total4 + e];
      q = make_float4(q.x + qx.x, q.y + qx.y, q.z + qx.z, q.w + qx.w);
      k = make_float4(k.x + kx.x, k.y + kx.y, k.z + kx.z, k.w + kx.w);
    }
    store_grad4(dqv, b, 0, t, d, make_float4(q.x * scale, q.y * scale, q.z * scale, q.w * scale));
    store_grad4(dkv, b, 0, t, d, k);
  }
}


// ---------------------------------------------------------------------------------------------
// Decode step: one new query per head (position t-1) over a key cache of t keys. HBM-bound: every
// cached K and V row is read once. grid (ceil(t / chunk), nseq * heads): a workgroup takes one
// head over `chunk` keys (a multiple of 256 the host picks so that the grid fills the chip),
// wavefront w the keys [w chunk/4, (w+1) chunk/4) of that range, DEC_STEP keys at a time.
//
// Lane layout: lane = (row slot kq, column slice dc), LPK = D / (elements per 16 bytes) lanes per
// cached row, so one 16-byte load instruction reads 64 / LPK whole rows, contiguous in HBM. A lane
// holds its slice of q and, per step, NR rows of K and the same NR rows of V (both issued before
// any arithmetic). The NR partial dot products reduce over the LPK lanes of a row by a
// reduce-scatter (log2 NR exchange rounds that halve the values a lane carries), after which lane
// (kq, dc) holds the full logit of row slot kq of load dc / (LPK / NR). The wavefront then takes
// the step's maximum, rescales its running output when the maximum rises, passes the
// probabilities through LDS to the lanes holding the V rows, and adds p_j v_j into each lane's
// column slice. The wavefronts' partials (max, sum, output) merge in LDS; one partial per
// workgroup goes to the workspace. The group's selector head writes the updated selection to the
// workspace's state rows; decode_finish_kernel merges the partials and copies the state rows over
// the caller's state after every head has read the old one (a kernel boundary later).

constexpr int DEC_NR = 8;   // cached rows of K (and of V) per lane per step, at most
template <typename E, int D>
struct DecLayout {
  static constexpr int EPC = 16 / (int)sizeof(E);   // elements per 16-byte load
  static constexpr int LPK = D / EPC;                // lanes per cached row
  static constexpr int KPI = 64 / LPK;               // rows per load instruction
  static constexpr int NR = LPK < DEC_NR ? LPK : DEC_NR;   // rows per lane per step (K, V each)
  static constexpr int DUP = LPK / NR;               // lanes holding one logit after the reduction
  static constexpr int STEP = KPI * NR;              // keys per wavefront step
};

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}
template <typename E>
__device__ __forceinline__ float to_f32(E x) {
  if constexpr (sizeof(E) == 2) return __uint_as_float(((uint32_t)x) << 16);
  else return x;
}

template <typename E, int D>
__global__ __launch_bounds__(NTHREADS) void decode_partial_kernel(
    const E* __restrict__ q, const E* __restrict__ k, const E* __restrict__ v, const float* __restrict__ selected,
    int64_t state_ld, float* __restrict__ pm, float* __restrict__ pl, float* __restrict__ po,
    float* __restrict__ next_state, int heads, int groups, int t, int64_t kvs, int exempt, float scale, int chunk,
    int nchunk) {
  using L = DecLayout<E, D>;
  constexpr int EPC = L::EPC, LPK = L::LPK, KPI = L::KPI, NR = L::NR, DUP = L::DUP, STEP = L::STEP;
  union Row {
    uint4 u;
    E e[EPC];
  };
  __shared__ __align__(16) float sP[NWAVES][STEP];
  __shared__ float sPart[NWAVES][D + 2];

  const int cidx = blockIdx.x;
  const int64_t row = blockIdx.y;             // b * heads + head
  const int per = heads / groups;
  const int b = (int)(row / heads), hd = (int)(row % heads);
  const int64_t sg = (int64_t)b * groups + hd / per;
  const bool selector = (hd % per) == 0;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int kq = lane / LPK, dc = lane % LPK;
  const int ri = dc / DUP;                    // after the reduction: the logit of row kq of load ri
  const bool owner = dc % DUP == 0;           // one lane per logit writes it
  const int wkeys = chunk / NWAVES;
  const int kw0 = cidx * chunk + wave * wkeys;
  const int kw_end = min(kw0 + wkeys, t);
  const float* selrow = selected + sg * state_ld;
  float* nextrow = next_state + sg * t;

  float qf[EPC];
  {
    Row qq;
    qq.u = *reinterpret_cast<const uint4*>(q + row * D + EPC * dc);
#pragma unroll
    for (int e = 0; e < EPC; ++e) qf[e] = to_f32(qq.e[e]) * scale;
  }
  // buffer resources over the head's t cached rows: the loads take one lane offset (row slot and
  // column slice) plus a wavefront-uniform offset of the rows, and rows at or past t read as zero
  constexpr int RB = D * (int)sizeof(E);   // bytes per cached row
  const int nbytes = t * RB;               // < 2^31 (rows_fit, checked by the C ABI)
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)(k + row * kvs), 0, nbytes, RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(v + row * kvs), 0, nbytes, RSRC_WORD3);
  const int loff = kq * RB + EPC * dc * (int)sizeof(E);
  float m = -INFINITY, l = 0.f, o[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) o[e] = 0.f;

  for (int kw = kw0; kw < kw_end; kw += STEP) {
    Row kr[NR], vr[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(krs, loff, (kw + i * KPI) * RB, 0);
      kr[i].u = make_uint4(x[0], x[1], x[2], x[3]);
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(vrs, loff, (kw + i * KPI) * RB, 0);
      vr[i].u = make_uint4(x[0], x[1], x[2], x[3]);
    }
    const int j = kw + ri * KPI + kq;         // this lane's logit after the reduction
    const bool jok = j < t;
    const float sel = jok ? selrow[j] : 0.f;
    float a[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < EPC; ++e) s = fmaf(qf[e], to_f32(kr[i].e[e]), s);
      a[i] = s;
    }
    // reduce-scatter over the row's lanes: the round with lane bit `s` keeps the upper half of the
    // values on lanes with the bit set, the lower half on the others, and adds the partner's copy
#pragma unroll
    for (int st = 1; st < NR; st <<= 1) {   // st = 1, 2, ..., NR/2: constant trip count, unrolled
      const int half = NR / (2 * st), s = LPK / (2 * st);
      // all-ones on lanes with the bit: a bitwise select (a ?: on the array elements becomes a
      // dynamically indexed read of the array)
      const uint32_t up = (lane & s) ? 0xffffffffu : 0u;
#pragma unroll
      for (int i = 0; i < half; ++i) {
        const uint32_t lo = __float_as_uint(a[i]), hi = __float_as_uint(a[i + half]);
        const float send = __uint_as_float((lo & up) | (hi & ~up));
        const float keep = __uint_as_float((hi & up) | (lo & ~up));
        a[i] = keep + __shfl_xor(send, s);
      }
    }
#pragma unroll
    for (int s = DUP / 2; s >= 1; s >>= 1) a[0] += __shfl_xor(a[0], s);
    const float raw = a[0];
    if (selector && owner && j >= exempt && j < t - 1) nextrow[j] = sel + fmaxf(raw, 0.f);
    const float z = jok ? (raw - sel) * LOG2E : -INFINITY;
    const float m_new = fmaxf(m, wave_max(z));   // finite: a step's first key is < t
    const float alpha = fast_exp2(m - m_new);    // 0 on the first step (m = -inf)
    const float p = jok ? fast_exp2(z - m_new) : 0.f;
    l = fmaf(l, alpha, owner ? p : 0.f);         // per lane; summed over the wavefront at the end
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] *= alpha;
    m = m_new;
    if (owner) sP[wave][kq * NR + ri] = p;
    lds_wave_sync();
    float pr[NR];
#pragma unroll
    for (int i = 0; i < NR; i += 4) {
      const float4 p4 = *reinterpret_cast<const float4*>(&sP[wave][kq * NR + i]);
      pr[i] = p4.x;
      pr[i + 1] = p4.y;
      pr[i + 2] = p4.z;
      pr[i + 3] = p4.w;
    }
    lds_wave_sync();   // sP is rewritten next step
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
      for (int e = 0; e < EPC; ++e) o[e] = fmaf(pr[i], to_f32(vr[i].e[e]), o[e]);
  }
  l = wave_sum(l);
#pragma unroll
  for (int sh = LPK; sh < 64; sh <<= 1)
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] += __shfl_xor(o[e], sh);
  if (kq == 0) {
#pragma unroll
    for (int e = 0; e < EPC; ++e) sPart[wave][2 + EPC * dc + e] = o[e];
  }
  if (lane == 0) {
    sPart[wave][0] = m;   // -inf for a wavefront with no key (its l and o are 0)
    sPart[wave][1] = l;
  }
  __syncthreads();
  // merge the wavefronts' partials: wavefront 0, lanes over D + 2
  if (wave == 0) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) mx = fmaxf(mx, sPart[w][0]);
    const int64_t slot = row * nchunk + cidx;
    for (int c = lane; c < D + 2; c += 64) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < NWAVES; ++w) {
        const float wt = sPart[w][0] == -INFINITY ? 0.f : fast_exp2(sPart[w][0] - mx);
        acc = fmaf(wt, sPart[w][c], acc);
      }
      if (c == 0) pm[slot] = mx;
      else if (c == 1) pl[slot] = acc;
      else po[slot * D + c - 2] = acc;
    }
  }
}

// Blocks [0, rows): out[row] = the row's partials merged, sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M)
// l_p. Thread i first takes the maxima and sums of partials i, i + 256, ... (the weights go to LDS),
// then thread (slot, column quad) the output quads of partials slot, slot + 1024/D, ..., a batch of
// DEC_FIN_UNROLL loads in flight at a time; slots reduce over lanes and then over wavefronts.
// Blocks from `rows` on: selected[g][j] = the selector heads' updates (rows of t in next_state),
// exempt <= j < t - 1, `sblocks` blocks of 1024 keys per state row.
constexpr int DEC_FIN_UNROLL = 8;
constexpr int DEC_FIN_MAXPARTS = 4096;   // LDS weights of one row: nparts <= this

template <int D>
__global__ __launch_bounds__(NTHREADS) void decode_finish_kernel(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ po, float* __restrict__ out,
    int nparts, int rows, float* __restrict__ selected, const float* __restrict__ next_state, int64_t state_ld, int t,
    int exempt, int sblocks) {
  constexpr int QPP = D / 4;               // float4 quads per partial
  constexpr int SLOTS = NTHREADS / QPP;    // partials in flight per load instruction
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  if ((int)blockIdx.x >= rows) {
    const int s = (int)blockIdx.x - rows;
    const int64_t g = s / sblocks;
    const int j0 = (s % sblocks) * (4 * NTHREADS);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u * NTHREADS + tid;
      if (j >= exempt && j < t - 1) selected[g * state_ld + j] = next_state[g * t + j];
    }
    return;
  }
  __shared__ float sW[DEC_FIN_MAXPARTS];
  __shared__ float sRed[NWAVES];
  __shared__ float4 sO[NWAVES][QPP];
  const int64_t row = blockIdx.x;
  const float* rm = pm + row * nparts;
  const float* rl = pl + row * nparts;
  const float4* ro = reinterpret_cast<const float4*>(po + row * nparts * (int64_t)D);

  float mx = -INFINITY;
  for (int i = tid; i < nparts; i += NTHREADS) {
    const float m = rm[i];
    sW[i] = m;
    mx = fmaxf(mx, m);
  }
  mx = wave_max(mx);
  if (lane == 0) sRed[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(sRed[0], sRed[1]), fmaxf(sRed[2], sRed[3]));   // finite: every partial has a key
  __syncthreads();   // sRed is reused below
  float l = 0.f;
  for (int i = tid; i < nparts; i += NTHREADS) {
    const float w = fast_exp2(sW[i] - mx);
    sW[i] = w;
    l = fmaf(w, rl[i], l);
  }
  l = wave_sum(l);
  if (lane == 0) sRed[wave] = l;
  __syncthreads();
  l = sRed[0] + sRed[1] + sRed[2] + sRed[3];

  const int slot = tid / QPP, cq = tid % QPP;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int i0 = slot; i0 < nparts; i0 += SLOTS * DEC_FIN_UNROLL) {
    float4 x[DEC_FIN_UNROLL];
#pragma unroll
    for (int u = 0; u < DEC_FIN_UNROLL; ++u) {
      const int i = i0 + u * SLOTS;
      x[u] = i < nparts ? ro[(int64_t)i * QPP + cq] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < DEC_FIN_UNROLL; ++u) {
      const int i = i0 + u * SLOTS;
      const float w = i < nparts ? sW[i] : 0.f;
      acc.x = fmaf(w, x[u].x, acc.x);
      acc.y = fmaf(w, x[u].y, acc.y);
      acc.z = fmaf(w, x[u].z, acc.z);
      acc.w = fmaf(w, x[u].w, acc.w);
    }
  }
#pragma unroll
  for (int sh = QPP; sh < 64; sh <<= 1) {
    acc.x += __shfl_xor(acc.x, sh);
    acc.y += __shfl_xor(acc.y, sh);
    acc.z += __shfl_xor(acc.z, sh);
    acc.w += __shfl_xor(acc.w, sh);
  }
  if (lane < QPP) sO[wave][lane] = acc;
  __syncthreads();
  if (tid < QPP) {
    float4 o = sO[0][tid];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) {
      o.x += sO[w][tid].x;
      o.y += sO[w][tid].y;
      o.z += sO[w][tid].z;
      o.w += sO[w][tid].w;
    }
    const float inv = 1.f / l;
    reinterpret_cast<float4*>(out + row * D)[tid] = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
  }
}

// ---------------------------------------------------------------------------------------------
// Host side: launch sequences of one storage dtype and head dim.

template <class OP, int D>
int run_selection(const FwdCall& c, hipStream_t st) {
  using elem = typename OP::elem;
  const int NBq = (int)cdiv(c.Tq, TILE), NKT = (int)cdiv(c.Tk, TILE);
  TimedLaunch timed(SA_KERNEL_SELECTION, st);
  if constexpr (sizeof(elem) == 2 && D == 64) {
    const int64_t wgs = cdiv(NKT, NWAVES * SEL_CARRY_KPW);
    // (its carry stores address one sequence's plane through a 32-bit buffer range)
    if (wgs * c.nseq >= SEL_CARRY_MIN_BLOCKS && (int64_t)NBq * c.Tk * 4 < ((int64_t)1 << 31)) {
      hipLaunchKernelGGL(sel_carry64_kernel, dim3((unsigned)wgs, (unsigned)c.nseq), dim3(NTHREADS), 0,
                         st, static_cast<const uint16_t*>(c.q), static_cast<const uint16_t*>(c.k), c.carry,
                         c.state_in, c.state_out, c.state_ld, c.Tq, c.Tk, c.qs, c.ks, c.q_off, c.exempt, c.scale);
      return launch_status();
    }
  }
  const int RB = SEL_RB;
  dim3 g1((unsigned)cdiv(NKT, NWAVES), (unsigned)cdiv(NBq, RB), (unsigned)c.nseq);
  hipLaunchKernelGGL((sel_colsum_kernel<OP, D>), g1, dim3(NTHREADS), 0, st, static_cast<const elem*>(c.q),
                     static_cast<const elem*>(c.k), c.carry, c.H, c.Tq, c.Tk, c.qs, c.ks, c.q_off, c.exempt, c.scale,
                     RB);
  dim3 g2((unsigned)cdiv(c.Tk, NTHREADS), (unsigned)c.nseq);
  hipLaunchKernelGGL(sel_scan_kernel, g2, dim3(NTHREADS), 0, st, c.carry, c.state_in, c.state_out, c.state_ld, NBq,
                     c.Tk, c.q_off);
  return launch_status();
}

template <class OP, int D, int G>
void launch_fwd(const FwdCall& c, const typename OP::elem* vt, int64_t ldv) {   // vt: V^T (fwd_kernel only)
  using elem = typename OP::elem;
  const int NBq = (int)cdiv(c.Tq, TILE);
  dim3 grid((unsigned)cdiv(NBq, NWAVES), (unsigned)(c.nseq * (c.H / G)));
  // the layout of sa_forward: q contiguous, k rows D apart, k's sequences H heads apart
  const bool cv = c.qs.row == D && c.qs.head == (int64_t)c.Tq * D && c.qs.seq == (int64_t)c.H * c.qs.head &&
                  c.ks.row == D && c.ks.seq == (int64_t)c.H * c.ks.head;
  TimedLaunch timed(SA_KERNEL_FORWARD, c.st);
  if constexpr (sizeof(elem) == 2 && D == 64 && G <= 2) {   // the direct-load kernel
#define SA_LAUNCH_FWD64(CVV)                                                                                      \
  hipLaunchKernelGGL((fwd64_kernel<CVV, G>), grid, dim3(NTHREADS), 0, c.st, static_cast<const elem*>(c.q),       \
                     static_cast<const elem*>(c.k), static_cast<const elem*>(c.v), c.carry, c.out, c.rmax,        \
                     c.rden, static_cast<elem*>(c.y), c.ys, c.H, c.Tq, c.Tk, c.qs, c.ks, c.vs, c.q_off, c.exempt, \
                     c.scale, c.damp_mode, c.train_len)
    if (cv) SA_LAUNCH_FWD64(true);
    else SA_LAUNCH_FWD64(false);
#undef SA_LAUNCH_FWD64
  } else {
#define SA_LAUNCH_FWD(CVV)                                                                                        \
  hipLaunchKernelGGL((fwd_kernel<OP, D, G, CVV>), grid, dim3(NTHREADS), 0, c.st, static_cast<const elem*>(c.q),  \
                     static_cast<const elem*>(c.k), vt, c.carry, c.out, c.rmax, c.rden, static_cast<elem*>(c.y),  \
                     c.ys, c.H, c.Tq, c.Tk, c.qs, c.ks, c.q_off, ldv, c.exempt, c.scale, c.damp_mode, c.train_len)
    if (cv) SA_LAUNCH_FWD(true);
    else SA_LAUNCH_FWD(false);
#undef SA_LAUNCH_FWD
  }
}

template <class OP, int D>
int forward_impl(const FwdCall& c) {
  using elem = typename OP::elem;
  const int64_t ldv = sa_transposed_ld(c.Tk);
  elem* vt = static_cast<elem*>(c.ws);
  const int dtype = sizeof(elem) == 2 ? SA_DTYPE_BF16 : SA_DTYPE_F32;
  int G = auto_group(dtype, D, c.H, c.group, false);
  if constexpr (sizeof(elem) == 2 && D == 64) {
    if (c.group <= 0 && G == 2) G = fwd64_group(c.nseq, c.H, c.Tq, device_cus());
  }
  // V^T for fwd_kernel (fwd64_kernel, bf16 at head dim 64 with G <= 2, reads the V rows transposed
  // from LDS)
  if (!(sizeof(elem) == 2 && D == 64 && G <= 2))
    launch_transpose<elem, D>(static_cast<const elem*>(c.v), vt, c.Tk, ldv, c.vs, c.H, (int64_t)c.nseq * c.H, c.st);
  int rc = run_selection<OP, D>(c, c.st);
  if (rc) return rc;
  if (G == 4) {
    if constexpr (sizeof(elem) == 2 && D <= 64) launch_fwd<OP, D, 4>(c, vt, ldv);
  } else if (G == 2) {
    if constexpr (sizeof(elem) == 2 && D <= 64) launch_fwd<OP, D, 2>(c, vt, ldv);
  } else {
    launch_fwd<OP, D, 1>(c, vt, ldv);
  }
  return launch_status();
}

// Launch of the key-side kernel from its arguments (the grid as launch_bwd's).
template <class OP, int D, int G, bool CV>
void launch_kv_from(const KvLaunch& a) {
  using elem = typename OP::elem;
  dim3 grid((unsigned)cdiv(a.T, NWAVES * TILE), (unsigned)(a.nseq * (a.H / G)));
  hipLaunchKernelGGL((bwd_kv_kernel<OP, D, G, CV>), grid, dim3(NTHREADS), 0, a.st, static_cast<const elem*>(a.q),
                     static_cast<const elem*>(a.k), static_cast<const elem*>(a.v), static_cast<const elem*>(a.qt),
                     static_cast<const elem*>(a.dout), static_cast<const elem*>(a.dot), a.qs, a.ks, a.vs, a.dos, a.lse,
                     a.dbar, a.carry, a.ucheck, a.dk0h, a.dk0x, a.dkv, a.dvv, a.nseq, a.H, a.T, a.ldt, a.exempt,
                     a.scale);
}

template <bool CV, bool SOLO>
void launch_kv64_from(const KvLaunch& a) {
  dim3 grid((unsigned)cdiv(a.T, NWAVES * TILE), (unsigned)(a.nseq * a.H));
  hipLaunchKernelGGL((bwd_kv64_kernel<CV, SOLO>), grid, dim3(NTHREADS), 0, a.st, static_cast<const uint16_t*>(a.q),
                     static_cast<const uint16_t*>(a.k), static_cast<const uint16_t*>(a.v),
                     static_cast<const uint16_t*>(a.dout), a.qs, a.ks, a.vs, a.dos, a.lse, a.dbar, a.carry, a.ucheck,
                     a.dk0h, a.dk0x, a.dkv, a.dvv, a.nseq, a.H, a.T, a.ldt, a.exempt, a.scale);
}

// The two backward kernels; returns the launch status.
template <class OP, int D, int G>
int launch_bwd(const BwdCall& c, const typename OP::elem* qt, const typename OP::elem* kt,
                const typename OP::elem* dot, const float* lse, const float* dbar, float* ucheck, float* dq0h,
                float* dk0h, float* dq0x, float* dk0x, int64_t ldt) {
  using elem = typename OP::elem;
  const elem* q = static_cast<const elem*>(c.q);
  const elem* k = static_cast<const elem*>(c.k);
  const elem* v = static_cast<const elem*>(c.v);
  const elem* dout = static_cast<const elem*>(c.dout);
  dim3 grid((unsigned)cdiv(c.T, NWAVES * TILE), (unsigned)(c.nseq * (c.H / G)));
  // every view the contiguous (nseq, H, T, D) layout of sa_backward
  auto contiguous = [&](const Strides& s) {
    return s.row == D && s.head == (int64_t)c.T * D && s.seq == (int64_t)c.H * s.head;
  };
  const bool cv = contiguous(c.qs) && contiguous(c.ks) && contiguous(c.vs) && contiguous(c.dos);
  const int f32 = c.grad_dtype == SA_DTYPE_F32;
  const GradView dqv{c.dq, c.dqs, f32}, dkv{c.dk, c.dks, f32}, dvv{c.dv, c.dvs, f32};
  const KvLaunch kv{q,    k,       v,      qt,   dout, dot,    c.qs, c.ks, c.vs, c.dos,    lse,      dbar,
                    c.carry, ucheck, dk0h, dk0x, dkv,  dvv,    c.nseq, c.H,  c.T,  ldt,      c.exempt, c.scale,
                    c.st};
  // bf16: the key-side kernel's instances live in a translation unit of their own (sa_bf16_kv.hip)
  auto launch_kv = [&](bool cvv) -> int {
    if constexpr (sizeof(elem) == 2) {
      return launch_bwd_kv_bf16(D, G, cvv, kv);
    } else {
      if (cvv) launch_kv_from<OP, D, G, true>(kv);
      else launch_kv_from<OP, D, G, false>(kv);
      return launch_status();
    }
  };
#define SA_LAUNCH_DQ(CVV)                                                                                         \
  hipLaunchKernelGGL((bwd_dq_kernel<OP, D, G, CVV>), grid, dim3(NTHREADS), 0, c.st, q, k, v, kt, dout, c.qs, c.ks, \
                     c.vs, c.dos, lse, dbar, c.carry, ucheck, dq0h, dq0x, dqv, c.nseq, c.H, c.T, ldt, c.exempt,   \
                     c.scale)
  {
    TimedLaunch timed(SA_KERNEL_BACKWARD, c.st);
    const int rc = launch_kv(cv);
    if (rc) return rc;
  }
  {
    TimedLaunch timed(SA_KERNEL_BACKWARD_DQ, c.st);
    if constexpr (sizeof(elem) == 2 && D == 64 && G == 1) {   // one head per wavefront: the pipelined kernel
      const dim3 grid64((unsigned)cdiv(c.T, DQ64_WAVES * TILE), (unsigned)(c.nseq * c.H));
#define SA_LAUNCH_DQ64(CVV, SOLO, SNAKE)                                                                           \
  hipLaunchKernelGGL((bwd_dq64_kernel<CVV, SOLO, SNAKE>), grid64, dim3(DQ64_WAVES * 64), 0, c.st, q, k, v, dout, c.qs, \
                     c.ks, c.vs, c.dos, lse, dbar, c.carry, ucheck, dq0h, dq0x, dqv, c.nseq, c.H, c.T, ldt, c.exempt, \
                     c.scale, dq_slots)
      const int dq_slots = bwd_snake_slots((int64_t)grid64.x * grid64.y, 1, device_cus());
      if (c.H == 1) {   // one-head sequences: head 0's loop only
        if (cv) SA_LAUNCH_DQ64(true, true, false);
        else SA_LAUNCH_DQ64(false, true, false);
      } else if (dq_slots > 0) {
        if (cv) SA_LAUNCH_DQ64(true, false, true);
        else SA_LAUNCH_DQ64(false, false, true);
      } else {
        if (cv) SA_LAUNCH_DQ64(true, false, false);
        else SA_LAUNCH_DQ64(false, false, false);
      }
#undef SA_LAUNCH_DQ64
    } else {
      if (cv) SA_LAUNCH_DQ(true);
      else SA_LAUNCH_DQ(false);
    }
  }
#undef SA_LAUNCH_DQ
  return launch_status();
}

template <class OP, int D>
int backward_impl(const BwdCall& c) {
  using elem = typename OP::elem;
  const int nseq = c.nseq, H = c.H, T = c.T;
  const hipStream_t st = c.st;
  const int dtype = sizeof(elem) == 2 ? SA_DTYPE_BF16 : SA_DTYPE_F32;
  const int G = bwd_group(dtype, D, H, c.group);
  const int64_t R = (int64_t)nseq * H, ldt = sa_transposed_ld(T);
  const BwdLayout L = bwd_layout(nseq, H, T, D, sizeof(elem), G);
  char* base = static_cast<char*>(c.ws);
  elem* qt = reinterpret_cast<elem*>(base + L.qt);
  elem* dot = reinterpret_cast<elem*>(base + L.dot);
  elem* kt = reinterpret_cast<elem*>(base + L.kt);
  float* lse = reinterpret_cast<float*>(base + L.lse);
  float* dbar = reinterpret_cast<float*>(base + L.dbar);
  float* dq0h = reinterpret_cast<float*>(base + L.dq);
  float* dk0h = reinterpret_cast<float*>(base + L.dk);
  float* dq0x = reinterpret_cast<float*>(base + L.dq0x);
  float* dk0x = reinterpret_cast<float*>(base + L.dk0x);
  float* ucheck = reinterpret_cast<float*>(base + L.ucheck);
  const elem* q = static_cast<const elem*>(c.q);
  const elem* k = static_cast<const elem*>(c.k);
  const elem* dout = static_cast<const elem*>(c.dout);

  // bf16 at head dim 64 the backward kernels read their Q, dO and K rows transposed from LDS
  // (bwd_kv64_kernel, bwd_dq64_kernel): no transposed copies
  if constexpr (!(sizeof(elem) == 2 && D == 64)) {
    launch_transpose<elem, D>(q, qt, T, ldt, c.qs, H, R, st);
    launch_transpose<elem, D>(dout, dot, T, ldt, c.dos, H, R, st);
    launch_transpose<elem, D>(k, kt, T, ldt, c.ks, H, R, st);
  }
  hipLaunchKernelGGL((bwd_rowstats_kernel<OP, D>), dim3((unsigned)cdiv(R * ldt * (D / 8), NTHREADS)),
                     dim3(NTHREADS), 0, st, dout, c.dos, H, T, c.out, c.rmax, c.rden, lse, dbar, ldt, R * ldt);
  int rc = launch_status();   // the transposes and row statistics
  if (rc) return rc;
#define SA_LAUNCH_BWD(GG) launch_bwd<OP, D, GG>(c, qt, kt, dot, lse, dbar, ucheck, dq0h, dk0h, dq0x, dk0x, ldt)
  if constexpr (sizeof(elem) == 2 && D <= 32) {
    rc = (G == 2) ? SA_LAUNCH_BWD(2) : SA_LAUNCH_BWD(1);
  } else {
    rc = SA_LAUNCH_BWD(1);
  }
#undef SA_LAUNCH_BWD
  if (rc) return rc;
  if (H == 1) return SA_OK;   // a one-head sequence's kernels wrote its gradients to the views
  // head 0's dQ, dK: its own sums plus the other groups' shares
  const int64_t total4 = (int64_t)nseq * T * D / 4;
  const int f32 = c.grad_dtype == SA_DTYPE_F32;
  hipLaunchKernelGGL(bwd_finish_kernel, dim3((unsigned)std::min<int64_t>(cdiv(total4, NTHREADS), 8192)),
                     dim3(NTHREADS), 0, st, reinterpret_cast<const float4*>(dq0h),
                     reinterpret_cast<const float4*>(dk0h), reinterpret_cast<const float4*>(dq0x),
                     reinterpret_cast<const float4*>(dk0x), H / G - 1, GradView{c.dq, c.dqs, f32},
                     GradView{c.dk, c.dks, f32}, D,
                     (int64_t)T * D, total4, c.scale);
  return launch_status();
}

// Keys per decode workgroup: the smallest power of two from 256 up that keeps the grid at or under
// 2048 workgroups (8 per CU) up to 4096 keys, and beyond that as far as a row's partials need to
// fit decode_finish_kernel's LDS.
inline int decode_chunk(int64_t rows, int64_t t) {
  int64_t chunk = 256;
  while ((chunk < 4096 && rows * cdiv(t, chunk) > 2048) || cdiv(t, chunk) > DEC_FIN_MAXPARTS) chunk *= 2;
  return (int)chunk;
}

template <class OP, int D>
int decode_impl(const DecCall& c) {
  using elem = typename OP::elem;
  const int64_t rows = (int64_t)c.nseq * c.heads;
  const int chunk = decode_chunk(rows, c.t);
  const int nchunk = (int)cdiv(c.t, chunk);
  if (nchunk > DEC_FIN_MAXPARTS) return SA_ERR_ARGUMENT;
  // workspace: maxima, sums (rows * nchunk each, padded to 4) and outputs (rows * nchunk * D) of the
  // partials, then the updated selection rows
  const int64_t np = align_up(rows * nchunk, 4);
  float* pm = static_cast<float*>(c.ws);
  float* pl = pm + np;
  float* po = pl + np;
  float* next_state = pm + decode_partials_floats(c.nseq, c.heads, c.t, D);
  dim3 g1((unsigned)nchunk, (unsigned)rows);
  {
    TimedLaunch timed(c.timed ? SA_KERNEL_DECODE : -1, c.st);
    hipLaunchKernelGGL((decode_partial_kernel<elem, D>), g1, dim3(NTHREADS), 0, c.st, static_cast<const elem*>(c.q),
                       static_cast<const elem*>(c.k), static_cast<const elem*>(c.v), c.selected, c.state_ld, pm, pl,
                       po, next_state, c.heads, c.groups, c.t, c.kvs, c.exempt, c.scale, chunk, nchunk);
  }
  const int sblocks = (int)cdiv(c.t, 4 * NTHREADS);
  const int64_t nblocks = rows + (int64_t)c.nseq * c.groups * sblocks;
  hipLaunchKernelGGL((decode_finish_kernel<D>), dim3((unsigned)nblocks), dim3(NTHREADS), 0, c.st, pm, pl, po, c.out,
                     nchunk, (int)rows, c.selected, next_state, c.state_ld, c.t, c.exempt, sblocks);
  return launch_status();
}

template <class OP>
int decode_entry(const DecCall& c) {
  if (c.head_dim == 32) return decode_impl<OP, 32>(c);
  if (c.head_dim == 64) return decode_impl<OP, 64>(c);
  return decode_impl<OP, 128>(c);
}

template <class OP>
int forward_entry(const FwdCall& c) {
  if (c.head_dim == 32) return forward_impl<OP, 32>(c);
  if (c.head_dim == 64) return forward_impl<OP, 64>(c);
  return forward_impl<OP, 128>(c);
}

template <class OP>
int backward_entry(const BwdCall& c) {
  if (c.head_dim == 32) return backward_impl<OP, 32>(c);
  if (c.head_dim == 64) return backward_impl<OP, 64>(c);
  return backward_impl<OP, 128>(c);
}

}  // namespace

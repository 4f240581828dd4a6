// Host-side pieces shared by the translation units of libsa_hip.so (sa_abi.hip, sa_bf16.hip,
// sa_f32.hip): tile geometry, head grouping, workspace layout, argument checks, launch timing, and
// the entry points of the two storage dtypes, which live in their own translation units so that
// each is compiled with the code-generation options that suit it.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

#include "sa.h"

#define SA_HIDDEN __attribute__((visibility("hidden")))

namespace sa_host {

constexpr int TILE = 32;      // tile edge and carry checkpoint spacing (queries)
constexpr int NTHREADS = 256;
constexpr int NWAVES = 4;

// Event timing of the main kernels, for measurement tools (sa_timing_enable / sa_timing_read).
// Off by default; when on, each timed launch is bracketed by a pair of HIP events recorded on the
// launch's own stream. The registry is the only mutable host state of the library.
struct TimingRegistry {
  std::mutex mu;
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events[SA_KERNEL_COUNT];
};
TimingRegistry& timing();   // the one registry (sa_abi.hip)

// Brackets one launch: construct before it, destroy after it (both on stream st). A negative
// kernel id records nothing (callers that must not create events).
class TimedLaunch {
 public:
  TimedLaunch(int kernel, hipStream_t st) : kernel_(kernel), st_(st) {
    if (kernel_ < 0) return;
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

// Heads per wavefront of the forward (a group shares head 0's selection work: its logits, F):
// 4 at head dim <= 32, 2 at 64 (two heads' output sums in registers leave two workgroups per CU,
// which measures faster than three with one head), 1 beyond; fp32 storage 1.
inline int auto_group(int dtype, int64_t D, int64_t heads, int requested, bool backward) {
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

// Heads per wavefront of the bf16 head-dim-64 forward when the caller leaves the choice open and
// auto_group allows two. Two heads per wavefront share head 0's selection and run two workgroups per
// CU; one head per wavefront runs three per CU with half the work per workgroup, and gives the same
// bits (fwd64_kernel). Two win once their grid needs more than one round of workgroups (more than two
// per CU): the dispatch order (part_block) then balances the XCDs and the cheaper head-tiles tell.
// With one round or less the launch lasts about as long as its longest workgroup -- the last query
// rows' sweep over every key -- which one head per wavefront halves. Measured on MI355X (forward call,
// ms, one / two heads per wavefront, B x H x T): 1x16x16384 1.27 / 0.99, 1x12x16384 0.90 / 0.71,
// 2x12x8192 0.46 / 0.36, 4x16x4096 0.33 / 0.27 (more than one round); 1x8x16384 0.61 / 0.65,
// 1x16x8192 0.31 / 0.33, 1x12x8192 0.28 / 0.32, 2x12x4096 0.15 / 0.17, 1x2x16384 0.50 / 0.62 (one
// round or less).
inline int fwd64_group(int64_t nseq, int64_t heads, int64_t tq, int cus) {
  if (heads % 2 != 0) return 1;
  const int64_t workgroups = nseq * (heads / 2) * cdiv(cdiv(tq, TILE), NWAVES);
  return workgroups > 2 * (int64_t)cus ? 2 : 1;
}

// The dispatch order of the query-side backward kernel at head dim 64 (work_order_block): the number
// of its workgroups an XCD runs at once when a launch holds 2.7 to 3 of them per slot, where the
// order that follows each XCD's first round with its shortest workgroups balances the slots better
// (a list-scheduling simulation: 1.03x the balanced share against 1.11x at 3.0; measured at the 12
// heads of d768: 1.28 -> 1.18 ms); else 0, the longest-first order, which is already balanced at
// whole even numbers of rounds and better everywhere else that was simulated (head counts 2-40 at
// 8192 and 16384 tokens).
inline int bwd_snake_slots(int64_t workgroups, int per_cu, int cus) {
  const int64_t slots = (int64_t)(cus / 8) * per_cu;
  if (slots <= 0) return 0;
  const double rounds = (double)workgroups / (8.0 * (double)slots);
  return (rounds >= 2.7 && rounds <= 3.0) ? (int)slots : 0;
}

// Compute units of the current device (256 on MI355X, the figure used when the query fails).
inline int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();   // (the launches' status check reads the last error)
    return 256;
  }
  return n > 0 ? n : 256;
}

// Heads per wavefront of the backward kernels: a group shares head 0's selection work (its logits,
// the history F and the g products), so wider groups amortise it, within the register budget; by
// default one head (two heads per wavefront cost the second workgroup per CU, measured slower).
inline int bwd_group(int dtype, int64_t D, int64_t heads, int requested) {
  int g = requested > 0 ? requested : 1;
  const int cap = (dtype == SA_DTYPE_BF16 && D <= 32) ? 2 : 1;
  g = g > cap ? cap : g;
  while (g > 1 && (heads % g != 0)) g >>= 1;
  return g < 1 ? 1 : g;
}

struct BwdLayout {
  int64_t qt, dot, kt, lse, dbar, dq, dk, dq0x, dk0x, ucheck, total;
};

// Floats of one selection-suffix checkpoint plane: query block qb holds the keys of its causal
// part, [0, (qb + 1) * TILE), and the rows lie end to end (row qb at utri_row(qb)).
__host__ __device__ inline int64_t utri_row(int64_t qb) { return (TILE / 2) * qb * (qb + 1); }
__host__ __device__ inline int64_t utri_floats(int64_t NB) { return utri_row(NB); }

// Workspace of sa_backward: transposed Q, dO, K; row statistics; head 0's fp32 dQ, dK sums and
// its shares from the other groups, one slot per group (every other gradient goes straight to the
// caller's views); the selection-suffix checkpoints (one lower-triangular plane per head group and
// sequence).
inline BwdLayout bwd_layout(int64_t nseq, int64_t heads, int64_t t, int64_t D, int64_t esize, int64_t G) {
  const int64_t R = nseq * heads, ldt = sa_transposed_ld(t), NB = (t + TILE - 1) / TILE;
  BwdLayout L;
  int64_t off = 0;
  auto take = [&](int64_t bytes) { int64_t o = off; off = align_up(off + bytes, 256); return o; };
  // Q^T, dO^T, K^T: none at bf16 head dim 64, whose kernels read the Q, dO and K rows transposed
  // from LDS
  const int64_t tcopy = (esize == 2 && D == 64) ? 0 : R * D * ldt * esize;
  L.qt = take(tcopy);
  L.dot = take(tcopy);
  L.kt = take(tcopy);
  L.lse = take(R * ldt * 4);    // (R, ldt): rows padded per head
  L.dbar = take(R * ldt * 4);   // -dbar, likewise
  L.dq = take(nseq * t * D * 4);   // head 0's own fp32 sums (the other heads write their views)
  L.dk = take(nseq * t * D * 4);
  L.dq0x = take((heads / G - 1) * nseq * t * D * 4);   // groups 1 .. heads/G - 1: slots 0 ..
  L.dk0x = take((heads / G - 1) * nseq * t * D * 4);
  L.ucheck = take((heads / G) * nseq * utri_floats(NB) * 4);
  L.total = off;
  return L;
}

inline bool valid_dims(int64_t nseq, int64_t heads, int64_t t) {
  const int64_t lim = (int64_t)1 << 30;
  return nseq >= 1 && heads >= 1 && t >= 1 && nseq < 65536 && heads < 65536 && t < lim && nseq * heads < 65536;
}

// The kernels read one head's rows (and its transposed copies, rows padded to a multiple of 64)
// through buffer resources with 32-bit byte offsets: t rows `row` elements apart must stay below
// 2 GiB.
inline bool rows_fit(int64_t t, int64_t row, int dtype) {
  return (t + 64) * row * (dtype == SA_DTYPE_BF16 ? 2 : 4) < ((int64_t)1 << 31);
}


// Element strides of a (sequence, head, row) view of a tensor whose head_dim elements per row are
// contiguous: element (b, h, r, d) at p + b * seq + h * head + r * row + d.
// (The row stride is 32-bit: one head's rows span less than 2 GiB, rows_fit.)
struct Strides {
  int64_t seq, head;
  int row;
  __host__ __device__ int64_t at(int64_t b, int64_t h) const { return b * seq + h * head; }
};

// A gradient output view: element type fp32 (f32) or bf16, (sequence, head, row) strides.
struct GradView {
  void* p;
  Strides s;
  int f32;
};

// One sa_forward call after its checks (pointers already typed by the storage dtype's entry).
struct FwdCall {
  const void *q, *k, *v;
  Strides qs, ks, vs;   // q, k, v views
  void* y;              // optional storage-dtype copy of the output (NULL: none)
  Strides ys;
  float *out, *rmax, *rden, *carry;
  const float* state_in;
  float* state_out;
  int64_t state_ld;
  void* ws;
  int nseq, H, Tq, Tk;
  int q_off;
  float scale;
  int exempt, group, damp_mode;
  float train_len;
  int head_dim;
  hipStream_t st;
};

// One sa_backward call after its checks.
struct BwdCall {
  const void *q, *k, *v;
  Strides qs, ks, vs;
  const float* out;
  const void* dout;
  Strides dos;
  const float *rmax, *rden, *carry;
  void *dq, *dk, *dv, *ws;
  Strides dqs, dks, dvs;
  int nseq, H, T;
  float scale;
  int exempt, group, grad_dtype, head_dim;
  hipStream_t st;
};

// One sa_decode call after its checks.
struct DecCall {
  const void *q, *k, *v;
  float *out, *selected;
  int64_t state_ld;
  void* ws;
  int nseq, heads, groups, t;
  int64_t kvs;
  float scale;
  int exempt, head_dim;
  hipStream_t st;
  bool timed = true;   // false: no timing events (the allocation-free entry point)
};

// Workspace of sa_decode: the partials of (nseq*heads, chunks of 256 keys or more) fp32 maxima,
// sums (each padded to a multiple of 4) and D-wide outputs, then the updated selection,
// (nseq*groups, t) fp32 (groups <= heads).
inline int64_t decode_partials_floats(int64_t nseq, int64_t heads, int64_t t, int64_t D) {
  return align_up(nseq * heads * cdiv(t, 256), 4) * (D + 2);
}
inline int64_t decode_workspace_bytes(int64_t nseq, int64_t heads, int64_t t, int64_t D) {
  return align_up((decode_partials_floats(nseq, heads, t, D) + nseq * heads * t) * 4, 256);
}

// The key-side backward kernel's arguments, for a launch from another translation unit.
struct KvLaunch {
  const void *q, *k, *v, *qt, *dout, *dot;
  Strides qs, ks, vs, dos;
  const float *lse, *dbar, *carry;
  float *ucheck, *dk0h, *dk0x;
  GradView dkv, dvv;
  int nseq, H, T;
  int64_t ldt;
  int exempt;
  float scale;
  hipStream_t st;
};
SA_HIDDEN int launch_bwd_kv_bf16(int D, int G, bool cv, const KvLaunch& a);           // sa_bf16_kv.hip
SA_HIDDEN int launch_bwd_kv_bf16_generic(int D, int G, bool cv, const KvLaunch& a);   // sa_bf16_kvg.hip
SA_HIDDEN int launch_bwd_kv64_solo(bool cv, const KvLaunch& a);                       // sa_bf16_kv1.hip

SA_HIDDEN int forward_bf16(const FwdCall& c);    // sa_bf16.hip
SA_HIDDEN int backward_bf16(const BwdCall& c);
SA_HIDDEN int forward_f32(const FwdCall& c);     // sa_f32.hip
SA_HIDDEN int backward_f32(const BwdCall& c);
SA_HIDDEN int decode_bf16(const DecCall& c);     // sa_bf16_dec.hip
SA_HIDDEN int decode_f32(const DecCall& c);      // sa_f32.hip

}  // namespace sa_host

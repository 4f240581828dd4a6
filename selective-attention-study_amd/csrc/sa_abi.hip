// The C ABI of libsa_hip.so (include/sa.h): argument checks, workspace sizes, the timing
// registry, and dispatch to the bf16 / fp32 translation units.

#include <math.h>

#include "sa_host.h"

namespace sa_host {

TimingRegistry& timing() {
  static TimingRegistry r;
  return r;
}

}  // namespace sa_host

using namespace sa_host;

// ---------------------------------------------------------------------------------------------
// C ABI

extern "C" {

int sa_abi_version(void) { return 5; }

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
    case SA_ERR_SCRATCH: return "the decode step needs more scratch than sa_decode_noalloc's fixed array holds";
    default: return "unknown status";
  }
}

int64_t sa_transposed_ld(int64_t t) { return align_up(t < 1 ? 1 : t, 64); }

// The forward's scratch is the transposed value copy fwd_kernel reads; none where fwd64_kernel runs
// (bf16 at head dim 64, one or two heads per wavefront: it reads the V rows themselves).
int64_t sa_forward_workspace_bytes(int64_t nseq, int64_t heads, int64_t tk, int64_t head_dim, int dtype, int group) {
  const int64_t es = dtype == SA_DTYPE_BF16 ? 2 : 4;
  if (dtype == SA_DTYPE_BF16 && head_dim == 64 && auto_group(dtype, head_dim, heads, group, false) <= 2) return 0;
  return align_up(nseq * heads * head_dim * sa_transposed_ld(tk) * es, 256);
}

int sa_forward(const void* q, const void* k, const void* v, float* out, float* rmax, float* rden, float* carry,
               const float* state_in, float* state_out, int64_t state_ld, void* workspace,
               int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t tq, int64_t tk, int64_t q_offset,
               int64_t kv_stride, int64_t head_dim, float scale, int dtype, int exempt, int group, int damp_mode,
               int64_t train_len, void* stream) {
  if (!valid_dims(nseq, heads, tk) || tq < 1 || q_offset < 0 || q_offset + tq != tk) return SA_ERR_ARGUMENT;
  if (kv_stride == 0) kv_stride = tk * head_dim;
  if (kv_stride < tk * head_dim || kv_stride % 8 != 0) return SA_ERR_ARGUMENT;
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return SA_ERR_HEAD_DIM;
  const sa_view_strides qs{heads * tq * head_dim, tq * head_dim, head_dim};
  const sa_view_strides ks{heads * kv_stride, kv_stride, head_dim};
  return sa_forward_strided(q, &qs, k, &ks, v, &ks, out, nullptr, nullptr, rmax, rden, carry, state_in, state_out,
                            state_ld, workspace, workspace_bytes, nseq, heads, tq, tk, q_offset, head_dim, scale,
                            dtype, exempt, group, damp_mode, train_len, stream);
}

// A view's strides are usable by the kernels: non-negative, 16-byte multiples (rows are read in
// 16-byte chunks), and one head's rows (t + 64 of them, with the transposed copies' padding)
// within the 2 GiB a buffer resource addresses.
static bool view_ok(const sa_view_strides* s, int64_t t, int64_t head_dim, int dtype, bool output) {
  if (!s) return false;
  const int64_t epc = dtype == SA_DTYPE_BF16 ? 8 : 4;
  if (s->seq < 0 || s->head < 0 || s->row < head_dim) return false;
  if (s->seq % epc || s->head % epc || s->row % epc) return false;
  if (output && s->head < head_dim) return false;   // distinct heads of a row must not overlap
  return rows_fit(t, s->row, dtype);
}

int sa_forward_strided(const void* q, const sa_view_strides* q_strides, const void* k,
                       const sa_view_strides* k_strides, const void* v, const sa_view_strides* v_strides,
                       float* out, void* y, const sa_view_strides* y_strides, float* rmax, float* rden,
                       float* carry, const float* state_in, float* state_out, int64_t state_ld, void* workspace,
                       int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t tq, int64_t tk,
                       int64_t q_offset, int64_t head_dim, float scale, int dtype, int exempt, int group,
                       int damp_mode, int64_t train_len, void* stream) {
  if (!valid_dims(nseq, heads, tk) || tq < 1 || q_offset < 0 || q_offset + tq != tk) return SA_ERR_ARGUMENT;
  if (!q || !k || !v || !out || !rmax || !rden || !carry || !state_out) return SA_ERR_ARGUMENT;
  if (q_offset > 0 && !state_in) return SA_ERR_ARGUMENT;
  if (state_ld < tk || exempt < 1 || damp_mode < 0 || damp_mode > 2 || (damp_mode && train_len < 1))
    return SA_ERR_ARGUMENT;
  if (!(scale > 0.f) || !(scale < INFINITY)) return SA_ERR_ARGUMENT;
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return SA_ERR_HEAD_DIM;
  if (!view_ok(q_strides, tq, head_dim, dtype, false) || !view_ok(k_strides, tk, head_dim, dtype, false) ||
      !view_ok(v_strides, tk, head_dim, dtype, false) || (y && !view_ok(y_strides, tq, head_dim, dtype, true)))
    return SA_ERR_ARGUMENT;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)y) % 16) return SA_ERR_ARGUMENT;
  const int64_t need = sa_forward_workspace_bytes(nseq, heads, tk, head_dim, dtype, group);
  if (workspace_bytes < need || (need > 0 && !workspace)) return SA_ERR_WORKSPACE;
  auto st = [](const sa_view_strides* p) { return p ? Strides{p->seq, p->head, (int)p->row} : Strides{0, 0, 0}; };
  FwdCall c{};
  c.q = q;
  c.k = k;
  c.v = v;
  c.qs = st(q_strides);
  c.ks = st(k_strides);
  c.vs = st(v_strides);
  c.y = y;
  c.ys = st(y_strides);
  c.out = out;
  c.rmax = rmax;
  c.rden = rden;
  c.carry = carry;
  c.state_in = state_in;
  c.state_out = state_out;
  c.state_ld = state_ld;
  c.ws = workspace;
  c.nseq = (int)nseq;
  c.H = (int)heads;
  c.Tq = (int)tq;
  c.Tk = (int)tk;
  c.q_off = (int)q_offset;
  c.scale = scale;
  c.exempt = exempt;
  c.group = group;
  c.damp_mode = damp_mode;
  c.train_len = (float)train_len;
  c.head_dim = (int)head_dim;
  c.st = static_cast<hipStream_t>(stream);
  return dtype == SA_DTYPE_BF16 ? forward_bf16(c) : forward_f32(c);
}

int64_t sa_backward_workspace_bytes(int64_t nseq, int64_t heads, int64_t t, int64_t head_dim, int dtype, int group) {
  if (!valid_dims(nseq, heads, t) || (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F32)) return -1;
  return bwd_layout(nseq, heads, t, head_dim, dtype == SA_DTYPE_BF16 ? 2 : 4, bwd_group(dtype, head_dim, heads, group))
      .total;
}

int sa_backward(const void* q, const void* k, const void* v, const float* out, const void* dout, const float* rmax,
                const float* rden, const float* carry, void* dq, void* dk, void* dv, void* workspace,
                int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t t, int64_t head_dim, float scale,
                int dtype, int grad_dtype, int exempt, int group, void* stream) {
  const sa_view_strides c{heads * t * head_dim, t * head_dim, head_dim};
  return sa_backward_strided(q, &c, k, &c, v, &c, out, dout, &c, rmax, rden, carry, dq, &c, dk, &c, dv, &c,
                             workspace, workspace_bytes, nseq, heads, t, head_dim, scale, dtype, grad_dtype, exempt,
                             group, stream);
}

int sa_backward_strided(const void* q, const sa_view_strides* q_strides, const void* k,
                        const sa_view_strides* k_strides, const void* v, const sa_view_strides* v_strides,
                        const float* out, const void* dout, const sa_view_strides* dout_strides, const float* rmax,
                        const float* rden, const float* carry, void* dq, const sa_view_strides* dq_strides, void* dk,
                        const sa_view_strides* dk_strides, void* dv, const sa_view_strides* dv_strides,
                        void* workspace, int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t t,
                        int64_t head_dim, float scale, int dtype, int grad_dtype, int exempt, int group,
                        void* stream) {
  if (!valid_dims(nseq, heads, t) || exempt < 1) return SA_ERR_ARGUMENT;
  if (!(scale > 0.f) || !(scale < INFINITY)) return SA_ERR_ARGUMENT;
  if (!q || !k || !v || !out || !dout || !rmax || !rden || !carry || !dq || !dk || !dv || !workspace)
    return SA_ERR_ARGUMENT;
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (grad_dtype != SA_DTYPE_BF16 && grad_dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return SA_ERR_HEAD_DIM;
  if (!view_ok(q_strides, t, head_dim, dtype, false) || !view_ok(k_strides, t, head_dim, dtype, false) ||
      !view_ok(v_strides, t, head_dim, dtype, false) || !view_ok(dout_strides, t, head_dim, dtype, false) ||
      !view_ok(dq_strides, t, head_dim, grad_dtype, true) || !view_ok(dk_strides, t, head_dim, grad_dtype, true) ||
      !view_ok(dv_strides, t, head_dim, grad_dtype, true))
    return SA_ERR_ARGUMENT;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)dout | (uintptr_t)dq | (uintptr_t)dk | (uintptr_t)dv) %
      16)
    return SA_ERR_ARGUMENT;
  if (group < 0 || workspace_bytes < sa_backward_workspace_bytes(nseq, heads, t, head_dim, dtype, group))
    return SA_ERR_WORKSPACE;
  auto st = [](const sa_view_strides* p) { return Strides{p->seq, p->head, (int)p->row}; };
  BwdCall c{};
  c.q = q;
  c.k = k;
  c.v = v;
  c.qs = st(q_strides);
  c.ks = st(k_strides);
  c.vs = st(v_strides);
  c.out = out;
  c.dout = dout;
  c.dos = st(dout_strides);
  c.rmax = rmax;
  c.rden = rden;
  c.carry = carry;
  c.dq = dq;
  c.dk = dk;
  c.dv = dv;
  c.ws = workspace;
  c.dqs = st(dq_strides);
  c.dks = st(dk_strides);
  c.dvs = st(dv_strides);
  c.nseq = (int)nseq;
  c.H = (int)heads;
  c.T = (int)t;
  c.scale = scale;
  c.exempt = exempt;
  c.group = group;
  c.grad_dtype = grad_dtype;
  c.head_dim = (int)head_dim;
  c.st = static_cast<hipStream_t>(stream);
  return dtype == SA_DTYPE_BF16 ? backward_bf16(c) : backward_f32(c);
}

int64_t sa_decode_workspace_bytes(int64_t nseq, int64_t heads, int64_t t, int64_t head_dim) {
  if (!valid_dims(nseq, heads, t) || head_dim < 1) return -1;
  return decode_workspace_bytes(nseq, heads, t, head_dim);
}

// Argument checks of the decode step, shared by sa_decode and sa_decode_noalloc (all but the
// workspace); kv_stride 0 becomes t * head_dim.
static int decode_check(const void* q, const void* k, const void* v, const float* out, const float* selected,
                        int64_t state_ld, int64_t nseq, int64_t heads, int64_t groups, int64_t t,
                        int64_t& kv_stride, int64_t head_dim, float scale, int dtype, int exempt) {
  if (!valid_dims(nseq, heads, t) || groups < 1 || heads % groups != 0 || exempt < 1) return SA_ERR_ARGUMENT;
  if (!q || !k || !v || !out || !selected || state_ld < t) return SA_ERR_ARGUMENT;
  if (!(scale > 0.f) || !(scale < INFINITY)) return SA_ERR_ARGUMENT;
  if (dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F32) return SA_ERR_DTYPE;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return SA_ERR_HEAD_DIM;
  if (!rows_fit(t, head_dim, dtype)) return SA_ERR_ARGUMENT;
  if (kv_stride == 0) kv_stride = t * head_dim;
  if (kv_stride < t * head_dim || kv_stride % 8 != 0) return SA_ERR_ARGUMENT;
  return SA_OK;
}

static int decode_run(const void* q, const void* k, const void* v, float* out, float* selected, int64_t state_ld,
                      void* workspace, int64_t nseq, int64_t heads, int64_t groups, int64_t t, int64_t kv_stride,
                      int64_t head_dim, float scale, int dtype, int exempt, void* stream, bool timed) {
  DecCall c{q,         k,          v,           out,    selected,  state_ld, workspace,
            (int)nseq, (int)heads, (int)groups, (int)t, kv_stride, scale,    exempt,
            (int)head_dim, static_cast<hipStream_t>(stream)};
  c.timed = timed;
  return dtype == SA_DTYPE_BF16 ? decode_bf16(c) : decode_f32(c);
}

int sa_decode(const void* q, const void* k, const void* v, float* out, float* selected, int64_t state_ld,
              void* workspace, int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t groups, int64_t t,
              int64_t kv_stride, int64_t head_dim, float scale, int dtype, int exempt, void* stream) {
  const int rc = decode_check(q, k, v, out, selected, state_ld, nseq, heads, groups, t, kv_stride, head_dim, scale,
                              dtype, exempt);
  if (rc != SA_OK) return rc;
  if (!workspace) return SA_ERR_ARGUMENT;
  if (workspace_bytes < sa_decode_workspace_bytes(nseq, heads, t, head_dim)) return SA_ERR_WORKSPACE;
  return decode_run(q, k, v, out, selected, state_ld, workspace, nseq, heads, groups, t, kv_stride, head_dim, scale,
                    dtype, exempt, stream, true);
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Allocation-free decode: the step's scratch (partial softmax sums, the new state rows) lives in
// a file-scope device array instead of a workspace argument. Every GPU the library runs on holds
// its own copy of the array (at its own address) until the process ends. The host-side symbol
// `scratch` is not a device address: its address on a device comes from hipGetSymbolAddress, once
// per device with that device current, and only that address reaches kernels.

static __device__ __align__(256) unsigned char scratch[SA_DECODE_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_at[MAX_DEVICES];   // the array's address on each device, once looked up

// The array's address on the current device, looked up on the first call for that device.
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return SA_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_at[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SA_ERR_LAUNCH;
    scratch_at[dev] = p;
  }
  *out = scratch_at[dev];
  return SA_OK;
}

}  // namespace

extern "C" {

int sa_decode_noalloc(const void* q, const void* k, const void* v, float* out, float* selected, int64_t state_ld,
                      int64_t nseq, int64_t heads, int64_t groups, int64_t t, int64_t kv_stride, int64_t head_dim,
                      float scale, int dtype, int exempt, void* stream) {
  const int rc = decode_check(q, k, v, out, selected, state_ld, nseq, heads, groups, t, kv_stride, head_dim, scale,
                              dtype, exempt);
  if (rc != SA_OK) return rc;
  if (sa_decode_workspace_bytes(nseq, heads, t, head_dim) > SA_DECODE_SCRATCH_BYTES) return SA_ERR_SCRATCH;
  void* ws = nullptr;
  const int got = scratch_of_current_device(&ws);
  if (got != SA_OK) return got;
  // nothing in the scratch needs to start at zero: the partial kernel writes every partial and
  // state row the finishing kernel reads
  return decode_run(q, k, v, out, selected, state_ld, ws, nseq, heads, groups, t, kv_stride, head_dim, scale, dtype,
                    exempt, stream, false);
}

}  // extern "C"


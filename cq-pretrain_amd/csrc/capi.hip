// extern "C" entry points of libcqgdn (declared in include/cqgdn.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "cqgdn.h"
#include "gdn_kernels.hpp"
#include "gdn_layout.hpp"

using namespace cqgdn;

namespace {
thread_local std::string g_error;
}  // namespace

namespace cqgdn {
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return CQGDN_OK;
}
}  // namespace cqgdn

namespace {

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CQGDN_EHIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_common(int64_t T, int H, int64_t n_chunks, int n_docs, const int32_t* chunk_table,
                 const int32_t* doc_chunk) {
  if (T < 0 || H <= 0 || n_chunks < 0 || n_docs < 0)
    return fail(CQGDN_EINVAL, "invalid sizes T=%lld H=%d n_chunks=%lld n_docs=%d", (long long)T, H,
                (long long)n_chunks, n_docs);
  if (T > 0 && (n_chunks == 0 || n_docs == 0))
    return fail(CQGDN_EINVAL, "T=%lld events need at least one chunk and one document", (long long)T);
  if (n_chunks > 0 && (!chunk_table || !doc_chunk)) return fail(CQGDN_EINVAL, "chunk_table/doc_chunk are null");
  if (n_chunks > INT32_MAX / 2 || (int64_t)n_chunks * H > 2147483647LL)
    return fail(CQGDN_EUNSUPPORTED, "too many chunks (%lld)", (long long)n_chunks);
  return CQGDN_OK;
}

int fwd_impl(const void* q, const void* k, const void* v, const float* g, const float* beta, int64_t T, int H,
             const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs, float scale,
             unsigned flags, const float* initial_state, float* final_state, void* o, void* workspace,
             size_t workspace_bytes, void* stream, hipStream_t scan_stream = nullptr,
             hipEvent_t scan_fork = nullptr, hipEvent_t scan_join = nullptr);

// The workspace of cqgdn_fwd_static: one array per GPU, held until the process
// ends.  Host code never uses its name as an address (on the host it only
// stands for the symbol): each device's address is looked up once, with that
// device current, and kept in g_static_ws.
__device__ __align__(256) uint8_t scratch[CQGDN_STATIC_WORKSPACE_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_static_mu;
void* g_static_ws[kMaxDevices] = {};

// The side stream and its two events: cqgdn_bwd_recompute runs the forward scan
// on it, cqgdn_bwd its bwd_dkw beside the reverse scan.
// One set per (thread, device), created on first use and kept until the process
// ends.  Per thread, so that a caller capturing a HIP graph never shares them with
// another thread's calls.
struct ScanSide {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  int cus = 0;  // compute units of the device
};

int scan_side(ScanSide** out) {
  thread_local ScanSide sides[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(CQGDN_EHIP, "cqgdn_bwd_recompute: no current HIP device (or device %d >= %d)", dev, kMaxDevices);
  ScanSide& s = sides[dev];
  if (!s.stream) {
    // the events only order two streams of this device: no system-scope fence (its
    // cache write-back and invalidation cost the stream a gap of several microseconds
    // at each record)
    constexpr unsigned kFlags = hipEventDisableTiming | hipEventDisableSystemFence;
    hipError_t e = hipEventCreateWithFlags(&s.fork, kFlags);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.join, kFlags);
    // default priority (the caller's streams are too); non-blocking: no implicit
    // ordering against the null stream, the events order everything
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&s.cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) {
      s.stream = nullptr;
      return fail(CQGDN_EHIP, "cqgdn_bwd_recompute: creating its scan stream and events: %s", hipGetErrorString(e));
    }
  }
  *out = &s;
  return CQGDN_OK;
}

constexpr int kBesideMinChunks = 64;

// The side stream for a kernel beside a state scan, or null (*out) when that kernel
// runs after the scan: each scan workgroup (one per head, 16-wide value slice and
// document) holds a whole CU, and the kernel beside waits for the scan's chunks,
// so every scan workgroup must be resident at once, leaving at least half of the
// CUs to the kernel beside; `env` = "0" in the environment keeps the kernel after
// the scan.
int side_beside_scan(const char* env, int64_t T, int H, int64_t n_chunks, int n_docs, ScanSide** out) {
  *out = nullptr;
  const char* e = getenv(env);
  if ((e && e[0] == '0') || T <= 0 || H <= 0 || n_docs <= 0) return CQGDN_OK;
  // documents of fewer chunks than this on average: the scan is too short for
  // the side stream's extra launches and events to pay
  if (n_chunks < (int64_t)kBesideMinChunks * n_docs) return CQGDN_OK;
  ScanSide* side = nullptr;
  if (const int err = scan_side(&side)) return err;
  if ((int64_t)H * 8 * n_docs * 2 <= side->cus) *out = side;
  return CQGDN_OK;
}

int static_workspace(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(CQGDN_EHIP, "cqgdn_fwd_static: no current HIP device (or device %d >= %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_static_mu);
  if (!g_static_ws[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(CQGDN_EHIP, "cqgdn_fwd_static: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_static_ws[dev] = p;
  }
  *out = g_static_ws[dev];
  return CQGDN_OK;
}

}  // namespace

extern "C" {

const char* cqgdn_version(void) { return "cqgdn 0.1.0 gfx950"; }

const char* cqgdn_last_error(void) { return g_error.c_str(); }

int64_t cqgdn_chunk_table(const int64_t* bounds, int n_bounds, int32_t* table, int32_t* doc_chunk) {
  if (!bounds || n_bounds < 1 || bounds[0] != 0) {
    fail(CQGDN_EINVAL, "bounds must start at 0");
    return -1;
  }
  int64_t n = 0;
  for (int d = 0; d + 1 < n_bounds; ++d) {
    const int64_t a = bounds[d], b = bounds[d + 1];
    if (b < a) {
      fail(CQGDN_EINVAL, "bounds must be non-decreasing");
      return -1;
    }
    if (doc_chunk) doc_chunk[d] = (int32_t)n;
    for (int64_t s = a; s < b; s += CQGDN_CHUNK) {
      if (table) {
        table[2 * n] = (int32_t)s;
        table[2 * n + 1] = (int32_t)((b - s) < CQGDN_CHUNK ? (b - s) : CQGDN_CHUNK);
      }
      ++n;
    }
  }
  if (doc_chunk) doc_chunk[n_bounds - 1] = (int32_t)n;
  ok();
  return n;
}

size_t cqgdn_fwd_workspace_size(int64_t T, int H, int64_t n_chunks) {
  size_t s[F_COUNT], off[F_COUNT];
  fwd_sizes(T, H, n_chunks, s);
  return offsets(s, F_COUNT, off);
}

int cqgdn_fwd_buffer_offsets(int64_t T, int H, int64_t n_chunks, size_t* out, int count) {
  if (!out || count < F_COUNT) return fail(CQGDN_EINVAL, "need room for %d offsets", (int)F_COUNT);
  size_t s[F_COUNT];
  fwd_sizes(T, H, n_chunks, s);
  offsets(s, F_COUNT, out);
  return ok();
}

size_t cqgdn_bwd_workspace_size(int64_t T, int H, int64_t n_chunks) {
  size_t s[B_COUNT], off[B_COUNT];
  bwd_sizes(T, H, n_chunks, s);
  return offsets(s, B_COUNT, off);
}

int cqgdn_bwd_buffer_offsets(int64_t T, int H, int64_t n_chunks, size_t* out, int count) {
  if (!out || count < B_COUNT) return fail(CQGDN_EINVAL, "need room for %d offsets", (int)B_COUNT);
  size_t s[B_COUNT];
  bwd_sizes(T, H, n_chunks, s);
  offsets(s, B_COUNT, out);
  return ok();
}

int cqgdn_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta, int64_t T, int H,
              const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs, float scale,
              unsigned flags, const float* initial_state, float* final_state, void* o, void* workspace,
              size_t workspace_bytes, void* stream) {
  return fwd_impl(q, k, v, g, beta, T, H, chunk_table, n_chunks, doc_chunk, n_docs, scale, flags, initial_state,
                  final_state, o, workspace, workspace_bytes, stream);
}

int cqgdn_fwd_static_init(void) {
  void* ws = nullptr;
  return static_workspace(&ws);
}

int cqgdn_fwd_static(const void* q, const void* k, const void* v, const float* g, const float* beta, int64_t T,
                     int H, const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs,
                     float scale, unsigned flags, const float* initial_state, float* final_state, void* o,
                     void* stream) {
  if (const int e = check_common(T, H, n_chunks, n_docs, chunk_table, doc_chunk)) return e;
  if (flags & CQGDN_TRAINING)
    return fail(CQGDN_EINVAL, "cqgdn_fwd_static is an inference forward: its workspace does not outlive the call, "
                              "so it cannot feed cqgdn_bwd (CQGDN_TRAINING)");
  const size_t need = cqgdn_fwd_workspace_size(T, H, n_chunks);
  if (need > (size_t)CQGDN_STATIC_WORKSPACE_BYTES)
    return fail(CQGDN_EINVAL,
                "T=%lld events x H=%d heads need a %zu-byte workspace, more than the %zu-byte static one: use "
                "cqgdn_fwd with a caller workspace",
                (long long)T, H, need, (size_t)CQGDN_STATIC_WORKSPACE_BYTES);
  void* ws = nullptr;
  if (T > 0)
    if (const int e = static_workspace(&ws)) return e;
  return fwd_impl(q, k, v, g, beta, T, H, chunk_table, n_chunks, doc_chunk, n_docs, scale, flags, initial_state,
                  final_state, o, ws, need, stream);
}

}  // extern "C"

namespace {
int fwd_impl(const void* q, const void* k, const void* v, const float* g, const float* beta, int64_t T, int H,
             const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs, float scale,
             unsigned flags, const float* initial_state, float* final_state, void* o, void* workspace,
             size_t workspace_bytes, void* stream, hipStream_t scan_stream, hipEvent_t scan_fork,
             hipEvent_t scan_join) {
  if (const int e = check_common(T, H, n_chunks, n_docs, chunk_table, doc_chunk)) return e;
  if (flags & ~(CQGDN_NORMALIZE | CQGDN_TRAINING | CQGDN_PRECISE | CQGDN_NO_OUTPUT | CQGDN_FP16))
    return fail(CQGDN_EINVAL, "unknown flags 0x%x", flags);
  if ((flags & CQGDN_NO_OUTPUT) && !(flags & CQGDN_TRAINING))
    return fail(CQGDN_EINVAL, "CQGDN_NO_OUTPUT rebuilds a training workspace: it needs CQGDN_TRAINING");
  if ((flags & CQGDN_TRAINING) && (flags & CQGDN_PRECISE))
    return fail(CQGDN_EINVAL, "CQGDN_PRECISE is an inference forward: it cannot be combined with CQGDN_TRAINING");
  if ((flags & CQGDN_TRAINING) && (initial_state || final_state))
    return fail(CQGDN_EINVAL, "a CQGDN_TRAINING forward starts from a zero state and returns no final state "
                              "(as the reference's training adapter, ops/gated_delta_net.py:231-232)");
  if (T == 0) {
    if (final_state && n_docs > 0) {
      // every document is empty: its final state is its initial state (or zero)
      launch_copy_or_zero(final_state, initial_state, (size_t)n_docs * H * 128 * 128, (hipStream_t)stream);
      return check_launch("cqgdn_fwd (empty)");
    }
    return ok();
  }
  if (!q || !k || !v || !g || !beta || (!o && !(flags & CQGDN_NO_OUTPUT)) || !workspace)
    return fail(CQGDN_EINVAL, "null tensor pointer");
  const size_t need = cqgdn_fwd_workspace_size(T, H, n_chunks);
  if (workspace_bytes < need)
    return fail(CQGDN_EINVAL, "forward workspace too small: %zu < %zu bytes", workspace_bytes, need);
  if (!aligned(workspace, 256)) return fail(CQGDN_EINVAL, "workspace must be 256-byte aligned");
  for (const void* p : {q, k, v, (const void*)o})
    if (p && !aligned(p, 16)) return fail(CQGDN_EINVAL, "q/k/v/o must be 16-byte aligned");
  FwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.g = g;
  a.beta = beta;
  a.chunks = chunk_table;
  a.doc_chunk = doc_chunk;
  a.T = (int)T;
  a.H = H;
  a.n_chunks = (int)n_chunks;
  a.n_docs = n_docs;
  a.scale = scale;
  a.normalize = (flags & CQGDN_NORMALIZE) != 0;
  a.precise = (flags & CQGDN_PRECISE) != 0;
  a.fp16 = (flags & CQGDN_FP16) != 0;
  a.training = (flags & CQGDN_TRAINING) != 0;
  a.no_output = (flags & CQGDN_NO_OUTPUT) != 0;
  a.initial_state = initial_state;
  a.final_state = final_state;
  a.o = o;
  a.ws = static_cast<uint8_t*>(workspace);
  cqgdn_fwd_buffer_offsets(T, H, n_chunks, a.off, F_COUNT);
  a.scan_stream = scan_stream;
  a.scan_fork = scan_fork;
  a.scan_join = scan_join;
  if (const hipError_t e = launch_fwd(a, (hipStream_t)stream))
    return fail(CQGDN_EHIP, "cqgdn_fwd: ordering the state scan's stream: %s", hipGetErrorString(e));
  return check_launch("cqgdn_fwd");
}

// cqgdn_bwd's checks and launch; with launch == false only the checks (for a caller
// that must know the backward's arguments are valid before it launches anything).
int bwd_impl(const void* q, const void* k, const void* v, const float* g, const float* beta, const void* dout,
             int64_t T, int H,
             const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs, float scale,
             unsigned flags, const void* fwd_workspace, size_t fwd_workspace_bytes, void* bwd_workspace,
             size_t bwd_workspace_bytes, void* dq, void* dk, void* dv, float* dg, float* dbeta, void* stream,
             bool launch, hipEvent_t dkw_after, hipStream_t side = nullptr, hipEvent_t side_fork = nullptr,
             hipEvent_t side_join = nullptr) {
  if (const int e = check_common(T, H, n_chunks, n_docs, chunk_table, doc_chunk)) return e;
  if (flags & ~(CQGDN_NORMALIZE | CQGDN_TRAINING | CQGDN_FP16)) return fail(CQGDN_EINVAL, "unknown flags 0x%x", flags);
  if (T == 0) return ok();
  if (!q || !k || !v || !g || !beta || !dout || !fwd_workspace || !bwd_workspace || !dq || !dk || !dv || !dg ||
      !dbeta)
    return fail(CQGDN_EINVAL, "null tensor pointer");
  const size_t fneed = cqgdn_fwd_workspace_size(T, H, n_chunks);
  const size_t bneed = cqgdn_bwd_workspace_size(T, H, n_chunks);
  if (fwd_workspace_bytes < fneed) return fail(CQGDN_EINVAL, "forward workspace too small: %zu < %zu", fwd_workspace_bytes, fneed);
  if (bwd_workspace_bytes < bneed) return fail(CQGDN_EINVAL, "backward workspace too small: %zu < %zu", bwd_workspace_bytes, bneed);
  if (!aligned(fwd_workspace, 256) || !aligned(bwd_workspace, 256)) return fail(CQGDN_EINVAL, "workspaces must be 256-byte aligned");
  for (const void* p : {q, k, v, dout, (const void*)dq, (const void*)dk, (const void*)dv})
    if (!aligned(p, 16)) return fail(CQGDN_EINVAL, "q/k/v/do/dq/dk/dv must be 16-byte aligned");
  if (!launch) return ok();
  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.g = g;
  a.beta = beta;
  a.chunks = chunk_table;
  a.doc_chunk = doc_chunk;
  a.T = (int)T;
  a.H = H;
  a.n_chunks = (int)n_chunks;
  a.n_docs = n_docs;
  a.scale = scale;
  a.normalize = (flags & CQGDN_NORMALIZE) != 0;
  a.fp16 = (flags & CQGDN_FP16) != 0;
  a.fws = static_cast<const uint8_t*>(fwd_workspace);
  a.bws = static_cast<uint8_t*>(bwd_workspace);
  cqgdn_fwd_buffer_offsets(T, H, n_chunks, a.foff, F_COUNT);
  cqgdn_bwd_buffer_offsets(T, H, n_chunks, a.boff, B_COUNT);
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.dg = dg;
  a.dbeta = dbeta;
  a.dkw_after = dkw_after;
  a.side = side;
  a.side_fork = side_fork;
  a.side_join = side_join;
  if (side) {
    const char* t = getenv("CQGDN_TEST_DKW_GIVE_UP");  // failure-handling tests only
    a.dkw_never_ready = t && t[0] == '1';
  }
  if (const hipError_t e = launch_bwd(a, (hipStream_t)stream))
    return fail(CQGDN_EHIP, "cqgdn_bwd: waiting for the forward scan's stream: %s", hipGetErrorString(e));
  return check_launch("cqgdn_bwd");
}

}  // namespace

extern "C" {

int cqgdn_bwd(const void* q, const void* k, const void* v, const float* g, const float* beta, const void* dout,
              int64_t T, int H, const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs,
              float scale, unsigned flags, const void* fwd_workspace, size_t fwd_workspace_bytes,
              void* bwd_workspace, size_t bwd_workspace_bytes, void* dq, void* dk, void* dv, float* dg, float* dbeta,
              void* stream) {
  // bwd_dkw beside the reverse scan when every scan workgroup is resident at once
  // (CQGDN_DKW_BESIDE_SCAN=0 keeps it after the scan); every argument is checked
  // before the side stream is looked up
  if (const int e = bwd_impl(q, k, v, g, beta, dout, T, H, chunk_table, n_chunks, doc_chunk, n_docs, scale, flags,
                             fwd_workspace, fwd_workspace_bytes, bwd_workspace, bwd_workspace_bytes, dq, dk, dv, dg,
                             dbeta, stream, false, nullptr))
    return e;
  ScanSide* side = nullptr;
  if (const int e = side_beside_scan("CQGDN_DKW_BESIDE_SCAN", T, H, n_chunks, n_docs, &side)) return e;
  return bwd_impl(q, k, v, g, beta, dout, T, H, chunk_table, n_chunks, doc_chunk, n_docs, scale, flags, fwd_workspace,
                  fwd_workspace_bytes, bwd_workspace, bwd_workspace_bytes, dq, dk, dv, dg, dbeta, stream, true,
                  nullptr, side ? side->stream : nullptr, side ? side->fork : nullptr, side ? side->join : nullptr);
}

int cqgdn_bwd_recompute(const void* q, const void* k, const void* v, const float* g, const float* beta,
                        const void* dout, int64_t T, int H, const int32_t* chunk_table, int64_t n_chunks,
                        const int32_t* doc_chunk, int n_docs, float scale, unsigned flags, void* fwd_workspace,
                        size_t fwd_workspace_bytes, void* bwd_workspace, size_t bwd_workspace_bytes, void* dq,
                        void* dk, void* dv, float* dg, float* dbeta, void* stream) {
  if (flags & ~(CQGDN_NORMALIZE | CQGDN_TRAINING | CQGDN_FP16))
    return fail(CQGDN_EINVAL, "unknown flags 0x%x", flags);
  // every argument is checked before anything is launched
  if (const int e = bwd_impl(q, k, v, g, beta, dout, T, H, chunk_table, n_chunks, doc_chunk, n_docs, scale, flags,
                             fwd_workspace, fwd_workspace_bytes, bwd_workspace, bwd_workspace_bytes, dq, dk, dv, dg,
                             dbeta, stream, false, nullptr))
    return e;
  if (T == 0) return ok();
  ScanSide* side = nullptr;
  if (const int e = scan_side(&side)) return e;
  const unsigned fflags = (flags & (CQGDN_NORMALIZE | CQGDN_FP16)) | CQGDN_TRAINING | CQGDN_NO_OUTPUT;
  if (const int e = fwd_impl(q, k, v, g, beta, T, H, chunk_table, n_chunks, doc_chunk, n_docs, scale, fflags, nullptr,
                             nullptr, nullptr, fwd_workspace, fwd_workspace_bytes, stream, side->stream, side->fork,
                             side->join))
    return e;
  return bwd_impl(q, k, v, g, beta, dout, T, H, chunk_table, n_chunks, doc_chunk, n_docs, scale, flags,
                  fwd_workspace, fwd_workspace_bytes, bwd_workspace, bwd_workspace_bytes, dq, dk, dv, dg, dbeta, stream,
                  true, side->join);
}

int cqgdn_recurrent(const void* q, const void* k, const void* v, const float* g, const void* beta, int dtype_flags,
                    float* state, void* out, int N, int E, int H, float scale, void* stream) {
  if (N < 0 || E < 0 || H <= 0) return fail(CQGDN_EINVAL, "invalid sizes N=%d E=%d H=%d", N, E, H);
  if (dtype_flags & ~(CQGDN_RECURRENT_BETA_BF16 | CQGDN_RECURRENT_FP16))
    return fail(CQGDN_EINVAL, "unknown dtype flags 0x%x", dtype_flags);
  if (N == 0 || E == 0) return ok();
  if (!q || !k || !v || !g || !beta || !state || !out) return fail(CQGDN_EINVAL, "null tensor pointer");
  for (const void* p : {q, k, (const void*)state})
    if (!aligned(p, 16)) return fail(CQGDN_EINVAL, "q/k/state must be 16-byte aligned");
  if ((int64_t)N * H * 2 > 2147483647LL) return fail(CQGDN_EUNSUPPORTED, "too many sequences");
  launch_recurrent(q, k, v, g, beta, (dtype_flags & CQGDN_RECURRENT_BETA_BF16) != 0,
                   (dtype_flags & CQGDN_RECURRENT_FP16) != 0, state, out, N, E, H, scale, (hipStream_t)stream);
  return check_launch("cqgdn_recurrent");
}

int cqgdn_l2norm_fwd(const void* x, void* y, float* rstd, int64_t rows, void* stream) {
  if (rows < 0) return fail(CQGDN_EINVAL, "rows < 0");
  if (rows == 0) return ok();
  if (!x || !y) return fail(CQGDN_EINVAL, "null tensor pointer");
  if (!aligned(x, 16) || !aligned(y, 16)) return fail(CQGDN_EINVAL, "x/y must be 16-byte aligned");
  launch_l2norm_fwd(static_cast<const bf16*>(x), static_cast<bf16*>(y), rstd, rows, (hipStream_t)stream);
  return check_launch("cqgdn_l2norm_fwd");
}

int cqgdn_l2norm_bwd(const void* y, const float* rstd, const void* dy, void* dx, int64_t rows, void* stream) {
  if (rows < 0) return fail(CQGDN_EINVAL, "rows < 0");
  if (rows == 0) return ok();
  if (!y || !rstd || !dy || !dx) return fail(CQGDN_EINVAL, "null tensor pointer");
  if (!aligned(y, 16) || !aligned(dy, 16) || !aligned(dx, 16)) return fail(CQGDN_EINVAL, "y/dy/dx must be 16-byte aligned");
  launch_l2norm_bwd(static_cast<const bf16*>(y), rstd, static_cast<const bf16*>(dy), static_cast<bf16*>(dx), rows,
                    (hipStream_t)stream);
  return check_launch("cqgdn_l2norm_bwd");
}

int cqgdn_chunk_local_cumsum(const float* g, float* out, int64_t T, int H, const int32_t* chunk_table,
                             int64_t n_chunks, int reverse, void* stream) {
  if (T < 0 || H <= 0 || n_chunks < 0) return fail(CQGDN_EINVAL, "invalid sizes");
  if (T == 0 || n_chunks == 0) return ok();
  if (!g || !out || !chunk_table) return fail(CQGDN_EINVAL, "null pointer");
  launch_chunk_cumsum(g, out, chunk_table, (int)n_chunks, H, reverse != 0, (hipStream_t)stream);
  return check_launch("cqgdn_chunk_local_cumsum");
}

namespace {
int check_conv(const void* x, const void* w, const int32_t* bounds, int n_docs, int64_t T, int C, int K) {
  if (T < 0 || n_docs < 0 || C <= 0) return fail(CQGDN_EINVAL, "invalid sizes T=%lld C=%d n_docs=%d", (long long)T, C, n_docs);
  if (K < 2 || K > 4) return fail(CQGDN_EUNSUPPORTED, "kernel width %d (2..4 supported)", K);
  if (C % 8) return fail(CQGDN_EUNSUPPORTED, "channels %d not a multiple of 8", C);
  if (T > INT32_MAX / 2 || (int64_t)C * T > ((int64_t)1 << 40)) return fail(CQGDN_EUNSUPPORTED, "too many rows");
  if (T > 0 && (!x || !w || !bounds || n_docs == 0)) return fail(CQGDN_EINVAL, "null pointer or no documents");
  if (!aligned(x, 16)) return fail(CQGDN_EINVAL, "x must be 16-byte aligned");
  return CQGDN_OK;
}
}  // namespace

int cqgdn_conv1d_fwd(const void* x, const void* weight, const int32_t* bounds, int n_docs, int64_t T, int C, int K,
                     int activation, void* y, void* stream) {
  if (const int e = check_conv(x, weight, bounds, n_docs, T, C, K)) return e;
  if (T == 0) return ok();
  if (!y || !aligned(y, 16)) return fail(CQGDN_EINVAL, "y must be a 16-byte aligned buffer");
  launch_conv_fwd(static_cast<const bf16*>(x), nullptr, C, static_cast<const bf16*>(weight), bounds, n_docs, (int)T, C,
                  K, activation != 0, static_cast<bf16*>(y), (hipStream_t)stream);
  return check_launch("cqgdn_conv1d_fwd");
}

size_t cqgdn_conv1d_bwd_workspace_size(int64_t T, int C, int K) {
  if (T <= 0 || C <= 0 || K <= 0) return 0;
  return (size_t)conv_strips(T) * (size_t)C * (size_t)K * sizeof(float);
}

int cqgdn_conv1d_bwd(const void* x, const void* weight, const void* dy, const int32_t* bounds, int n_docs, int64_t T,
                     int C, int K, int activation, void* dx, float* dweight, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (const int e = check_conv(x, weight, bounds, n_docs, T, C, K)) return e;
  if (T == 0) return ok();
  if (!dy || !dx || !dweight || !aligned(dy, 16) || !aligned(dx, 16))
    return fail(CQGDN_EINVAL, "dy/dx/dweight must be non-null (dy, dx 16-byte aligned)");
  if (!workspace || !aligned(workspace, 16) || workspace_bytes < cqgdn_conv1d_bwd_workspace_size(T, C, K))
    return fail(CQGDN_EINVAL, "workspace must be 16-byte aligned and >= cqgdn_conv1d_bwd_workspace_size bytes");
  launch_conv_bwd(static_cast<const bf16*>(x), nullptr, C, static_cast<const bf16*>(weight),
                  static_cast<const bf16*>(dy), bounds, n_docs, (int)T, C, K, activation != 0, static_cast<bf16*>(dx),
                  nullptr, C, dweight, static_cast<float*>(workspace), (hipStream_t)stream);
  return check_launch("cqgdn_conv1d_bwd");
}

size_t cqgdn_gated_norm_bwd_workspace_size(int64_t rows, int H) {
  if (rows <= 0 || H <= 0) return 0;
  return (size_t)gnorm_bwd_blocks(rows, H) * CQGDN_HEAD_DIM * sizeof(float);
}

namespace {
int check_gnorm(const void* y, int64_t rows, int H, const void* z, int64_t z_stride, const float* weight) {
  if (rows < 0 || H <= 0) return fail(CQGDN_EINVAL, "invalid sizes rows=%lld H=%d", (long long)rows, H);
  if (rows > 0 && (!y || !z || !weight)) return fail(CQGDN_EINVAL, "y, z and weight must be non-null");
  if (z_stride < (int64_t)H * CQGDN_HEAD_DIM || z_stride % 8)
    return fail(CQGDN_EINVAL, "z_stride=%lld must be >= H*128 and a multiple of 8", (long long)z_stride);
  if (!aligned(y, 16) || !aligned(z, 16) || !aligned(weight, 16))
    return fail(CQGDN_EINVAL, "y, z and weight must be 16-byte aligned");
  return CQGDN_OK;
}
}  // namespace

int cqgdn_gated_norm_fwd(const void* y, const int32_t* index, int64_t rows, int H, const void* z, int64_t z_stride,
                         const float* weight, float eps, void* out, float* rstd, void* stream) {
  if (const int e = check_gnorm(y, rows, H, z, z_stride, weight)) return e;
  if (rows == 0) return ok();
  if (!out || !rstd || !aligned(out, 16)) return fail(CQGDN_EINVAL, "out (16-byte aligned) and rstd must be non-null");
  launch_gnorm_fwd(static_cast<const bf16*>(y), index, rows, H, static_cast<const bf16*>(z), z_stride, weight, eps,
                   static_cast<bf16*>(out), rstd, (hipStream_t)stream);
  return check_launch("cqgdn_gated_norm_fwd");
}

int cqgdn_gated_norm_bwd(const void* y, const int32_t* index, const int32_t* zero_rows, int64_t n_zero, int64_t rows,
                         int H, const void* z, int64_t z_stride, const float* weight, const float* rstd,
                         const void* dout, void* dy, void* dz, int64_t dz_stride, float* dweight, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (const int e = check_gnorm(y, rows, H, z, z_stride, weight)) return e;
  if (n_zero < 0 || (n_zero > 0 && !zero_rows)) return fail(CQGDN_EINVAL, "zero_rows must hold n_zero >= 0 rows");
  if (rows == 0 && n_zero == 0) return ok();
  if (!dy || !dz || !dweight || !rstd || !dout || !aligned(dy, 16) || !aligned(dz, 16) || !aligned(dout, 16))
    return fail(CQGDN_EINVAL, "rstd, dout, dy, dz, dweight must be non-null (dout, dy, dz 16-byte aligned)");
  if (dz_stride < (int64_t)H * CQGDN_HEAD_DIM || dz_stride % 8)
    return fail(CQGDN_EINVAL, "dz_stride=%lld must be >= H*128 and a multiple of 8", (long long)dz_stride);
  if (rows > 0 && (!workspace || !aligned(workspace, 16) ||
                   workspace_bytes < cqgdn_gated_norm_bwd_workspace_size(rows, H)))
    return fail(CQGDN_EINVAL, "workspace must be 16-byte aligned and >= cqgdn_gated_norm_bwd_workspace_size bytes");
  launch_gnorm_bwd(static_cast<const bf16*>(y), index, zero_rows, n_zero, rows, H, static_cast<const bf16*>(z),
                   z_stride, weight, rstd, static_cast<const bf16*>(dout), static_cast<bf16*>(dy),
                   static_cast<bf16*>(dz), dz_stride, dweight, static_cast<float*>(workspace), (hipStream_t)stream);
  return check_launch("cqgdn_gated_norm_bwd");
}

namespace {
size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// log2(H / HK) for supported value and key head counts, -1 otherwise
int head_group_shift(int H, int HK) {
  auto pow2 = [](int x) { return x == 4 || x == 8 || x == 16 || x == 32; };
  if (!pow2(H) || !pow2(HK) || HK > H) return -1;
  int s = 0;
  while ((HK << s) < H) ++s;
  return s;
}

int ev_args(const cqgdn_event_plan* p, int H, int HK, const void* raw, int64_t raw_stride, const void* a,
            int64_t a_stride, const void* b, int64_t b_stride, const void* w, const float* A_log,
            const float* dt_bias, EvArgs& out) {
  if (!p) return fail(CQGDN_EINVAL, "plan is null");
  const int gshift = head_group_shift(H, HK);
  if (gshift < 0)
    return fail(CQGDN_EINVAL, "H=%d key_heads=%d: supported local heads are 4, 8, 16, 32, key heads dividing H", H, HK);
  if (p->n_content < 0 || p->n_queries < 0 || p->n_events < 0 || p->n_content_docs < 0 || p->n_history_rows < 0)
    return fail(CQGDN_EINVAL, "negative plan sizes");
  if (p->conv_kernel < 2 || p->conv_kernel > 4) return fail(CQGDN_EINVAL, "conv_kernel=%d not in 2..4", p->conv_kernel);
  const int64_t C = (int64_t)(2 * HK + H) * CQGDN_HEAD_DIM;
  if (raw_stride < C || raw_stride % 8)
    return fail(CQGDN_EINVAL, "raw_stride must be >= (2*key_heads + H)*128 and a multiple of 8");
  if (a_stride < H || b_stride < H) return fail(CQGDN_EINVAL, "a_stride and b_stride must be >= H");
  if (!raw || !a || !b || !w || !A_log || !dt_bias || !aligned(raw, 16))
    return fail(CQGDN_EINVAL, "raw (16-byte aligned), a, b, conv_weight, A_log, dt_bias must be non-null");
  if (p->n_events > 0 && (!p->event_q || !p->event_write))
    return fail(CQGDN_EINVAL, "event_q and event_write are null");
  if (p->n_content > 0 && (!p->content_order || !p->content_bounds || p->n_content_docs < 1 || !p->q_ptr ||
                           !p->q_list || !p->write_event || !p->history_ptr || !p->history_list))
    return fail(CQGDN_EINVAL, "content index arrays are null");
  if (p->n_queries > 0 && (!p->query_source || !p->query_history || !p->query_event))
    return fail(CQGDN_EINVAL, "query index arrays are null");
  if (p->n_history_rows > 0 && !p->history_rows) return fail(CQGDN_EINVAL, "history_rows is null");
  if (p->n_fold_rows < 0 || p->n_fold_rows > p->n_content ||
      (p->n_fold_rows > 0 && (!p->fold_rows || !p->fold_ptr || !p->fold_list)))
    return fail(CQGDN_EINVAL, "fold rows: n_fold_rows must be in 0..n_content with non-null fold arrays");
  out = EvArgs{H, HK, gshift, p->conv_kernel, p->n_content, p->n_queries, p->n_events, p->n_history_rows,
               p->content_order, p->event_q, p->event_write, p->query_source, p->query_history,
               p->q_ptr, p->q_list, p->write_event, p->query_event, p->history_ptr, p->history_list,
               p->history_rows, static_cast<const bf16*>(raw), raw_stride, static_cast<const bf16*>(a), a_stride,
               static_cast<const bf16*>(b), b_stride, static_cast<const bf16*>(w), A_log, dt_bias};
  return CQGDN_OK;
}
}  // namespace

size_t cqgdn_event_inputs_fwd_workspace_size(int n_content, int H, int key_heads) {
  if (n_content < 0 || H <= 0 || key_heads <= 0) return 0;
  return align256((size_t)n_content * (2 * key_heads + H) * CQGDN_HEAD_DIM * sizeof(bf16)) + 256;
}

int cqgdn_event_inputs_fwd(const cqgdn_event_plan* plan, int H, int key_heads, const void* raw, int64_t raw_stride,
                           const void* a, int64_t a_stride, const void* b, int64_t b_stride, const void* conv_weight,
                           const float* A_log, const float* dt_bias, void* q, void* k, void* v, float* g, float* beta,
                           void* workspace, size_t workspace_bytes, void* stream) {
  EvArgs ea;
  if (const int e = ev_args(plan, H, key_heads, raw, raw_stride, a, a_stride, b, b_stride, conv_weight, A_log,
                            dt_bias, ea))
    return e;
  if (plan->n_events > 0 && (!q || !k || !v || !g || !beta || !aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16)))
    return fail(CQGDN_EINVAL, "q, k, v (16-byte aligned), g, beta must be non-null");
  if (!workspace || !aligned(workspace, 256) ||
      workspace_bytes < cqgdn_event_inputs_fwd_workspace_size(plan->n_content, H, key_heads))
    return fail(CQGDN_EINVAL, "workspace must be 256-byte aligned and >= cqgdn_event_inputs_fwd_workspace_size");
  const int C = (2 * key_heads + H) * CQGDN_HEAD_DIM;
  bf16* conv = static_cast<bf16*>(workspace);
  hipStream_t st = (hipStream_t)stream;
  if (plan->n_content > 0)
    launch_conv_fwd(ea.raw, ea.order, raw_stride, ea.w, plan->content_bounds, plan->n_content_docs, plan->n_content,
                    C, plan->conv_kernel, 1, conv, st);
  launch_events_fwd(ea, conv, static_cast<bf16*>(q), static_cast<bf16*>(k), static_cast<bf16*>(v), g, beta, st);
  return check_launch("cqgdn_event_inputs_fwd");
}

namespace {
struct EvLayout {
  size_t dconv, dpre, gpart, qpart, cpart, qsum, dcont, dcgate, total;
};
EvLayout ev_layout(int n_content, int n_queries, int H, int HK, int K, bool fold) {
  const size_t SK = (size_t)HK * CQGDN_HEAD_DIM, C = 2 * SK + (size_t)H * CQGDN_HEAD_DIM;
  EvLayout l{};
  size_t o = 0;
  l.dcont = o; o += fold ? align256((size_t)n_content * C * sizeof(bf16)) : 0;
  l.dcgate = o; o += fold ? align256((size_t)n_content * 2 * H * sizeof(float)) : 0;
  l.dconv = o; o += align256((size_t)n_content * C * sizeof(bf16));
  l.dpre = o; o += align256((size_t)n_queries * SK * sizeof(float));
  l.gpart = o; o += align256((size_t)n_content * 2 * H * sizeof(float));
  l.qpart = o; o += align256((size_t)events_query_blocks(n_queries) * SK * K * sizeof(float));
  l.cpart = o; o += align256((size_t)(n_content > 0 ? conv_strips(n_content) : 0) * C * K * sizeof(float));
  l.qsum = o; o += align256(SK * K * sizeof(float));
  l.total = o + 256;
  return l;
}
}  // namespace

size_t cqgdn_event_inputs_bwd_workspace_size(const cqgdn_event_plan* plan, int H, int key_heads) {
  if (!plan || plan->n_content < 0 || plan->n_queries < 0 || H <= 0 || key_heads <= 0 || plan->conv_kernel < 2 ||
      plan->conv_kernel > 4)
    return 0;
  return ev_layout(plan->n_content, plan->n_queries, H, key_heads, plan->conv_kernel, plan->n_fold_rows > 0).total;
}

int cqgdn_event_inputs_bwd(const cqgdn_event_plan* plan, int H, int key_heads, const void* raw, int64_t raw_stride,
                           const void* a, int64_t a_stride, const void* b, int64_t b_stride, const void* conv_weight,
                           const float* A_log, const float* dt_bias, const void* dq, const void* dk, const void* dv,
                           const float* dg, const float* dbeta, void* d_raw, int64_t d_raw_stride, void* d_a,
                           int64_t d_a_stride, void* d_b, int64_t d_b_stride, float* dweight, float* dgate,
                           void* workspace, size_t workspace_bytes, void* stream) {
  EvArgs ea;
  if (const int e = ev_args(plan, H, key_heads, raw, raw_stride, a, a_stride, b, b_stride, conv_weight, A_log,
                            dt_bias, ea))
    return e;
  const int64_t C = (int64_t)(2 * key_heads + H) * CQGDN_HEAD_DIM;
  if (plan->n_events > 0 && (!dq || !dk || !dv || !dg || !dbeta || !aligned(dq, 16) || !aligned(dk, 16) ||
                             !aligned(dv, 16)))
    return fail(CQGDN_EINVAL, "dq, dk, dv (16-byte aligned), dg, dbeta must be non-null");
  if (!d_raw || !d_a || !d_b || !dweight || !dgate || !aligned(d_raw, 16) || !aligned(dweight, 16))
    return fail(CQGDN_EINVAL, "d_raw (16-byte aligned), d_a, d_b, dweight (16-byte aligned), dgate must be non-null");
  if (d_raw_stride < C || d_raw_stride % 8 || d_a_stride < H || d_b_stride < H)
    return fail(CQGDN_EINVAL, "gradient strides must match the input layouts");
  const bool fold = plan->n_fold_rows > 0;
  const EvLayout l = ev_layout(plan->n_content, plan->n_queries, H, key_heads, plan->conv_kernel, fold);
  if (!workspace || !aligned(workspace, 256) || workspace_bytes < l.total)
    return fail(CQGDN_EINVAL, "workspace must be 256-byte aligned and >= cqgdn_event_inputs_bwd_workspace_size");
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const EvGrads d{static_cast<const bf16*>(dq), static_cast<const bf16*>(dk), static_cast<const bf16*>(dv), dg, dbeta,
                  static_cast<bf16*>(d_raw), d_raw_stride, static_cast<bf16*>(d_a), d_a_stride,
                  static_cast<bf16*>(d_b), d_b_stride, dweight, dgate,
                  fold ? reinterpret_cast<bf16*>(ws + l.dcont) : nullptr,
                  fold ? reinterpret_cast<float*>(ws + l.dcgate) : nullptr, plan->n_fold_rows, plan->fold_rows,
                  plan->fold_ptr, plan->fold_list};
  const EvWork w{reinterpret_cast<bf16*>(ws + l.dconv), reinterpret_cast<float*>(ws + l.dpre),
                 reinterpret_cast<float*>(ws + l.gpart), reinterpret_cast<float*>(ws + l.qpart),
                 reinterpret_cast<float*>(ws + l.cpart), reinterpret_cast<float*>(ws + l.qsum)};
  launch_events_bwd(ea, d, plan->content_bounds, plan->n_content_docs, w, (hipStream_t)stream);
  return check_launch("cqgdn_event_inputs_bwd");
}

size_t cqgdn_layer_decode_workspace_size(int N, int H) {
  (void)N;
  (void)H;
  return 0;  // the step needs no workspace
}

int cqgdn_layer_decode_step(int N, int H, int key_heads, int conv_kernel, const void* proj, int64_t proj_stride,
                            void* conv_history, const void* conv_weight, const float* A_log, const float* dt_bias,
                            const float* norm_weight, float eps, float scale, float* state, void* out, void* workspace,
                            size_t workspace_bytes, void* stream) {
  const int gshift = head_group_shift(H, key_heads);
  if (N < 0 || gshift < 0 || conv_kernel < 2 || conv_kernel > 4)
    return fail(CQGDN_EINVAL, "invalid sizes N=%d H=%d key_heads=%d conv_kernel=%d", N, H, key_heads, conv_kernel);
  if (N == 0) return ok();
  const int64_t C = (int64_t)(2 * key_heads + H) * CQGDN_HEAD_DIM, SV = (int64_t)H * CQGDN_HEAD_DIM;
  if (proj_stride < C + SV + 2 * H || proj_stride % 8)
    return fail(CQGDN_EINVAL, "proj_stride must be >= (2*key_heads + 2*H)*128 + 2*H and a multiple of 8");
  if (!proj || !conv_history || !conv_weight || !A_log || !dt_bias || !norm_weight || !state || !out ||
      !aligned(proj, 16) || !aligned(conv_history, 16) || !aligned(out, 16) || !aligned(norm_weight, 16))
    return fail(CQGDN_EINVAL, "null or misaligned buffer (proj, conv_history, out, norm_weight need 16 bytes)");
  (void)workspace;  // none needed (see cqgdn_layer_decode_workspace_size)
  (void)workspace_bytes;
  hipStream_t st = (hipStream_t)stream;
  const DecArgs a{N, H, key_heads, gshift, conv_kernel, static_cast<const bf16*>(proj), proj_stride,
                  static_cast<bf16*>(conv_history),
                  static_cast<const bf16*>(conv_weight), A_log, dt_bias};
  launch_decode_step(a, state, norm_weight, eps, scale, static_cast<bf16*>(out), st);
  return check_launch("cqgdn_layer_decode_step");
}

}  // extern "C"

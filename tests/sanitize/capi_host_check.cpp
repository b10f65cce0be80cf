// Host-side checks of the libcqgdn C ABI, built with AddressSanitizer and
// UndefinedBehaviorSanitizer on the host code (tests/test_sanitize.py builds
// and runs it; no GPU is used: every call below either is host arithmetic or
// is rejected by the argument checks before any HIP call).
//
// Covered: the chunk table on exact-size heap buffers (an off-by-one write is
// a heap overflow), workspace sizes and buffer offsets over a grid of sizes
// (overflow of size arithmetic is undefined behaviour), and the rejection
// paths of every compute entry point, including long error messages.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

#include "cqgdn.h"

static int g_failures = 0;
#define CHECK(cond)                                                      \
  do {                                                                   \
    if (!(cond)) {                                                       \
      std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      ++g_failures;                                                      \
    }                                                                    \
  } while (0)

// exact-size heap copies, so that sanitizers see every out-of-bounds access
template <class T>
static std::unique_ptr<T[]> heap(const std::vector<T>& v) {
  std::unique_ptr<T[]> p(new T[v.size() ? v.size() : 1]);
  if (!v.empty()) std::memcpy(p.get(), v.data(), v.size() * sizeof(T));
  return p;
}

static void chunk_tables() {
  const std::vector<std::vector<int64_t>> cases = {
      {0}, {0, 0}, {0, 1}, {0, 64}, {0, 65}, {0, 0, 130, 130, 257, 257}, {0, 63, 64, 200, 1000}, {0, 9216}};
  for (const auto& b : cases) {
    auto bounds = heap(b);
    const int64_t n = cqgdn_chunk_table(bounds.get(), (int)b.size(), nullptr, nullptr);
    CHECK(n >= 0);
    int64_t expect = 0;
    for (size_t d = 0; d + 1 < b.size(); ++d) expect += (b[d + 1] - b[d] + CQGDN_CHUNK - 1) / CQGDN_CHUNK;
    CHECK(n == expect);
    std::unique_ptr<int32_t[]> table(new int32_t[2 * n + 1]), doc(new int32_t[b.size()]);
    CHECK(cqgdn_chunk_table(bounds.get(), (int)b.size(), table.get(), doc.get()) == n);
    for (int64_t c = 0; c < n; ++c) CHECK(table[2 * c + 1] >= 1 && table[2 * c + 1] <= CQGDN_CHUNK);
    CHECK(doc[b.size() - 1] == n);
  }
  const std::vector<int64_t> bad = {0, 10, 5};
  auto bb = heap(bad);
  CHECK(cqgdn_chunk_table(bb.get(), 3, nullptr, nullptr) == -1);
  const std::vector<int64_t> nonzero = {3, 10};
  auto nz = heap(nonzero);
  CHECK(cqgdn_chunk_table(nz.get(), 2, nullptr, nullptr) == -1);
  CHECK(cqgdn_chunk_table(nullptr, 2, nullptr, nullptr) == -1);
}

static void sizes_and_offsets() {
  for (int64_t T : {0LL, 1LL, 63LL, 64LL, 2304LL, 9216LL, 32768LL, 1LL << 22})
    for (int H : {4, 8, 16, 32}) {
      const int64_t nc = (T + CQGDN_CHUNK - 1) / CQGDN_CHUNK;
      const size_t fws = cqgdn_fwd_workspace_size(T, H, nc), bws = cqgdn_bwd_workspace_size(T, H, nc);
      std::unique_ptr<size_t[]> fo(new size_t[CQGDN_FWD_BUFFERS]), bo(new size_t[CQGDN_BWD_BUFFERS]);
      CHECK(cqgdn_fwd_buffer_offsets(T, H, nc, fo.get(), CQGDN_FWD_BUFFERS) == CQGDN_OK);
      CHECK(cqgdn_bwd_buffer_offsets(T, H, nc, bo.get(), CQGDN_BWD_BUFFERS) == CQGDN_OK);
      for (int i = 0; i < CQGDN_FWD_BUFFERS; ++i) CHECK(fo[i] % 256 == 0 && fo[i] <= fws);
      for (int i = 0; i < CQGDN_BWD_BUFFERS; ++i) CHECK(bo[i] % 256 == 0 && bo[i] <= bws);
      CHECK(cqgdn_fwd_buffer_offsets(T, H, nc, fo.get(), CQGDN_FWD_BUFFERS - 1) == CQGDN_EINVAL);
      (void)cqgdn_gated_norm_bwd_workspace_size(T, H);
      CHECK(cqgdn_conv1d_bwd_workspace_size(T, 3 * H * 128, 4) > 0 || T == 0);
      CHECK(cqgdn_layer_decode_workspace_size(64, H) == 0);
      CHECK(cqgdn_event_inputs_fwd_workspace_size((int)(T > 1 << 20 ? 1 << 20 : T), H, H) > 0);
    }
}

static void rejections() {
  // a fake device address: every call below must fail its argument checks first
  void* p = reinterpret_cast<void*>(uintptr_t{256});
  float* f = static_cast<float*>(p);
  int32_t* ip = static_cast<int32_t*>(p);
  const int32_t table[2] = {0, 64}, doc[2] = {0, 1};
  // cqgdn_fwd / cqgdn_fwd_static
  CHECK(cqgdn_fwd(p, p, p, f, f, 64, 12, table, 1, doc, 1, 1.f, CQGDN_TRAINING, nullptr, nullptr, p, p, 1 << 20,
                  nullptr) == CQGDN_EINVAL);  // H = 12
  CHECK(cqgdn_fwd(p, p, p, f, f, 64, 16, table, 1, doc, 1, 1.f, 0x80u, nullptr, nullptr, p, p, 1 << 20, nullptr) ==
        CQGDN_EINVAL);  // unknown flag
  CHECK(cqgdn_fwd(p, p, p, f, f, 64, 16, table, 1, doc, 1, 1.f, CQGDN_TRAINING, f, nullptr, p, p, 1 << 20,
                  nullptr) == CQGDN_EINVAL);  // training with an initial state
  CHECK(cqgdn_fwd(p, p, p, f, f, 64, 16, table, 1, doc, 1, 1.f, CQGDN_TRAINING, nullptr, nullptr, p, p, 16,
                  nullptr) == CQGDN_EINVAL);  // workspace too small
  CHECK(cqgdn_fwd(nullptr, p, p, f, f, 64, 16, table, 1, doc, 1, 1.f, 0, nullptr, nullptr, p, p, 1 << 30,
                  nullptr) == CQGDN_EINVAL);  // null q
  CHECK(cqgdn_fwd_static(p, p, p, f, f, 64, 16, table, 1, doc, 1, 1.f, CQGDN_TRAINING, nullptr, nullptr, p,
                         nullptr) == CQGDN_EINVAL);  // the static workspace serves no training
  CHECK(cqgdn_fwd_static(p, p, p, f, f, 1 << 20, 16, table, 1, doc, 1, 1.f, 0, nullptr, nullptr, p, nullptr) ==
        CQGDN_EINVAL);  // table inconsistent with T / larger than the static workspace
  // cqgdn_bwd
  CHECK(cqgdn_bwd(p, p, p, f, f, p, 64, 16, table, 1, doc, 1, 1.f, CQGDN_NORMALIZE | CQGDN_TRAINING, p, 16, p,
                  1 << 20, p, p, p, f, f, nullptr) == CQGDN_EINVAL);  // forward workspace too small
  CHECK(cqgdn_bwd(p, p, p, f, f, p, 64, 16, table, 1, doc, 1, 1.f, CQGDN_PRECISE, p, 1 << 30, p, 1 << 30, p, p, p,
                  f, f, nullptr) == CQGDN_EINVAL);  // flag not accepted by the backward
  CHECK(cqgdn_bwd(nullptr, p, p, f, f, p, 64, 16, table, 1, doc, 1, 1.f, CQGDN_NORMALIZE | CQGDN_TRAINING, p,
                  1 << 30, p, 1 << 30, p, p, p, f, f, nullptr) == CQGDN_EINVAL);  // q is read by the backward
  // recurrent, l2norm, cumsum, conv, gated norm
  CHECK(cqgdn_recurrent(p, p, p, f, p, 0, f, p, -1, 1, 16, 1.f, nullptr) == CQGDN_EINVAL);
  CHECK(cqgdn_recurrent(nullptr, p, p, f, p, 0, f, p, 1, 1, 16, 1.f, nullptr) == CQGDN_EINVAL);
  CHECK(cqgdn_l2norm_fwd(p, p, f, -1, nullptr) == CQGDN_EINVAL);
  CHECK(cqgdn_l2norm_bwd(nullptr, f, p, p, 4, nullptr) == CQGDN_EINVAL);
  CHECK(cqgdn_chunk_local_cumsum(nullptr, f, 4, 4, ip, 1, 0, nullptr) == CQGDN_EINVAL);
  CHECK(cqgdn_conv1d_fwd(p, p, ip, 1, 64, 100, 4, 1, p, nullptr) == CQGDN_EUNSUPPORTED);  // C not a multiple of 8
  CHECK(cqgdn_conv1d_fwd(p, p, ip, 1, 64, 128, 9, 1, p, nullptr) == CQGDN_EUNSUPPORTED);  // K out of range
  CHECK(cqgdn_conv1d_fwd(p, p, ip, 1, -1, 128, 4, 1, p, nullptr) == CQGDN_EINVAL);  // T < 0
  CHECK(cqgdn_gated_norm_fwd(nullptr, nullptr, 4, 16, p, 2048, f, 1e-6f, p, f, nullptr) == CQGDN_EINVAL);
  // the layer's event inputs and decode step
  cqgdn_event_plan plan;
  std::memset(&plan, 0, sizeof plan);
  plan.conv_kernel = 4;
  CHECK(cqgdn_event_inputs_fwd(&plan, 12, 12, p, 7000, p, 7000, p, 7000, p, f, f, p, p, p, f, f, p, 1 << 20,
                               nullptr) == CQGDN_EINVAL);  // H = 12
  CHECK(cqgdn_event_inputs_fwd(&plan, 16, 32, p, 7000, p, 7000, p, 7000, p, f, f, p, p, p, f, f, p, 1 << 20,
                               nullptr) == CQGDN_EINVAL);  // more key heads than value heads
  CHECK(cqgdn_event_inputs_fwd(&plan, 16, 16, p, 100, p, 7000, p, 7000, p, f, f, p, p, p, f, f, p, 1 << 20,
                               nullptr) == CQGDN_EINVAL);  // raw stride too small
  plan.conv_kernel = 7;
  CHECK(cqgdn_event_inputs_fwd(&plan, 16, 16, p, 6144, p, 6144, p, 6144, p, f, f, p, p, p, f, f, p, 1 << 20,
                               nullptr) == CQGDN_EINVAL);  // conv kernel out of range
  CHECK(cqgdn_event_inputs_bwd_workspace_size(&plan, 16, 16) == 0);
  plan.conv_kernel = 4;
  plan.n_fold_rows = -1;
  CHECK(cqgdn_event_inputs_bwd(&plan, 16, 16, p, 6144, p, 6144, p, 6144, p, f, f, p, p, p, f, f, p, 6144, p, 6144,
                               p, 6144, f, f, p, 1 << 20, nullptr) == CQGDN_EINVAL);  // fold rows < 0
  CHECK(cqgdn_event_inputs_fwd(nullptr, 16, 16, p, 6144, p, 6144, p, 6144, p, f, f, p, p, p, f, f, p, 1 << 20,
                               nullptr) == CQGDN_EINVAL);  // null plan
  CHECK(cqgdn_layer_decode_step(1, 32, 8, 4, p, 100, p, p, f, f, f, 1e-6f, 0.1f, f, p, nullptr, 0, nullptr) ==
        CQGDN_EINVAL);  // projection stride too small for the key heads
  CHECK(cqgdn_layer_decode_step(0, 32, 8, 4, p, 100, p, p, f, f, f, 1e-6f, 0.1f, f, p, nullptr, 0, nullptr) ==
        CQGDN_OK);  // nothing to do
  // every rejection leaves a message; long arguments format without overflow
  CHECK(cqgdn_timer_arm("a-kernel-name-that-does-not-exist-and-is-rather-long-xxxxxxxxxxxxxxxxxxxxxxxxxxxxxxxx", 4) ==
        CQGDN_EINVAL);
  CHECK(std::strstr(cqgdn_last_error(), "unknown kernel") != nullptr);
  CHECK(cqgdn_timer_arm("bwd_dkw", 0) == CQGDN_EINVAL);
  CHECK(std::strstr(cqgdn_last_error(), "max_launches") != nullptr);
  CHECK(cqgdn_timer_arm(nullptr, 0) == CQGDN_OK && cqgdn_last_error()[0] == 0);
  CHECK(std::strlen(cqgdn_version()) > 0);
}

int main() {
  chunk_tables();
  sizes_and_offsets();
  rejections();
  if (g_failures) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("capi host checks passed\n");
  return 0;
}

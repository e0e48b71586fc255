// Host-side argument validation of the C ABI under AddressSanitizer + UndefinedBehaviorSanitizer.
//
// Built from the library's sources with host code only (no device code, no GPU needed): every call
// below is one the library must reject, answer or fail on purpose before any HIP call, so the run
// exercises the validation, size-query, error-message and fault-injection paths of every entry.
// Exit status 0 when every check holds; the sanitizers abort the run on the first finding.
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "saf3r_hip.h"

static int g_failures = 0;

#define CHECK(cond)                                                                   \
  do {                                                                                \
    if (!(cond)) {                                                                    \
      std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      ++g_failures;                                                                   \
    }                                                                                 \
  } while (0)

// the last error names the entry and fits its buffer
static bool last_error_has(const char* part) {
  const char* e = saf3r_last_error();
  return e != nullptr && std::strlen(e) < 512 && std::strstr(e, part) != nullptr;
}

// an aligned non-null address that is never dereferenced on the host (device pointers are opaque here)
static void* fake(uintptr_t a = 256) { return reinterpret_cast<void*>(a); }

static void check_queries() {
  CHECK(saf3r_abi_version() == SAF3R_ABI_VERSION);
  CHECK(saf3r_packed_slots(128, 1374, 5) == 640 + 128 * 1408);
  CHECK(saf3r_packed_slots(0, 10, 1) == -1);
  CHECK(saf3r_packed_slots(2, 5, 5) == -1);
  CHECK(saf3r_packed_slots(-3, 1374, 5) == -1);
  CHECK(saf3r_packed_slots(INT_MAX, INT_MAX, 5) <= INT64_MAX);  // no signed overflow on the way
  CHECK(saf3r_packed_slots(1, 6, 5) > 0);

  CHECK(saf3r_token_topk_workspace_bytes(100, 4, 1369, 4) == 0);  // k <= 16: registers only
  CHECK(saf3r_token_topk_workspace_bytes(100, 4, 1369, 64) > 0);
  CHECK(saf3r_token_topk_workspace_bytes(0, 4, 1369, 64) == 0);
  CHECK(saf3r_token_topk_workspace_bytes(-1, 4, 1369, 64) == -1);
  CHECK(last_error_has("saf3r_token_topk_workspace_bytes"));
  CHECK(saf3r_token_topk_workspace_bytes(100, 4, 1369, 0) == -1);
  CHECK(saf3r_token_topk_workspace_bytes(100, 4, 1369, 129) == -1);
  CHECK(saf3r_token_topk_workspace_bytes(100, 4, 5000, 64) == -1);
  CHECK(saf3r_token_topk_workspace_bytes(INT_MAX, 65535, 4096, 128) >= 0);  // large, without overflow

  CHECK(saf3r_block_select_pooled_workspace_bytes(7, 128, 22, 4) == 0);  // no workspace
  CHECK(saf3r_block_select_pooled_workspace_bytes(7, 128, 22, 17) == 0);  // sequential kernel
  CHECK(saf3r_block_select_pooled_workspace_bytes(7, 128, 22, 0) == -1);
  CHECK(saf3r_block_select_pooled_workspace_bytes(7, 128, 33, 4) == -1);
  CHECK(saf3r_block_select_pooled_workspace_bytes(0, 128, 22, 4) == -1);
  CHECK(saf3r_block_select_pooled_workspace_bytes(65536, 128, 22, 4) == -1);  // more heads than the grid holds
  CHECK(saf3r_block_select_pooled_workspace_bytes(INT_MAX, INT_MAX, INT_MAX, INT_MAX) == -1);
}

static void check_sparse_attn() {
  const int32_t dense[2] = {SAF3R_DENSE, SAF3R_DENSE};
  void* d = fake();
  int rc = saf3r_sparse_attn_fwd(nullptr, nullptr, nullptr, 2, 100, 5, 2, dense, nullptr, 0, 0.125f, nullptr, 128,
                                 nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                                 nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("null"));
  const int32_t unknown[1] = {1000};
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, unknown, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("unknown pattern"));
  const int32_t keyset[1] = {SAF3R_KEYSET};
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, keyset, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("key-set"));
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, keyset, nullptr, 0, 0.125f, d, 64, d, d, static_cast<const int32_t*>(d), 100, nullptr,
                             nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("multiple of 64"));
  const int32_t bcast[1] = {SAF3R_BROADCAST};
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, bcast, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, d, d, nullptr, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("BROADCAST"));
  const int32_t dyn[1] = {SAF3R_BLOCK_DYNAMIC};
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, dyn, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("selection list"));
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, dyn, static_cast<const int32_t*>(d), 1 << 20, 0.125f, d, 64,
                             nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr,
                             0, nullptr);
  CHECK(rc == SAF3R_ERR_UNSUPPORTED && last_error_has("sel_width"));
  const uint8_t bad_layout[1] = {77};
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, dense, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, nullptr, nullptr, bad_layout, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("unknown layout"));
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, dense, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, nullptr, nullptr, nullptr, nullptr, 0x40, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("unknown flags"));
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 1, dense, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                             reinterpret_cast<unsigned long long*>(fake(260)), 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("8-byte aligned"));
  rc = saf3r_sparse_attn_fwd(d, d, d, 0, 100, 5, 1, dense, nullptr, 0, 0.125f, d, 64, nullptr, nullptr, nullptr, 0,
                             nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("geometry"));
  int32_t many[4096];
  for (int32_t& x : many) x = SAF3R_DENSE;
  rc = saf3r_sparse_attn_fwd(d, d, d, 2, 100, 5, 4096, many, nullptr, 0, 0.125f, d, 4096 * 64, nullptr, nullptr,
                             nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_UNSUPPORTED && last_error_has("num_heads"));
}

static void check_other_entries() {
  void* d = fake();
  const saf3r_rows rows = {d, 64, 0, 1 << 20, 0};
  const saf3r_rows null_rows = {nullptr, 64, 0, 1 << 20, 0};
  const saf3r_rows odd_rows = {fake(264), 64, 0, 1 << 20, 0};
  int32_t* di = static_cast<int32_t*>(d);
  float* df = static_cast<float*>(d);
  uint16_t* dh = static_cast<uint16_t*>(d);

  int rc = saf3r_pack_qkv(nullptr, d, d, 3072, 64, 4, 1374, 5, 16, nullptr, nullptr, nullptr, nullptr, 1e-6f, 0,
                          nullptr, nullptr, nullptr, 0, d, d, d, nullptr, nullptr, nullptr, nullptr, 1.f, nullptr,
                          nullptr, nullptr, nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("saf3r_pack_qkv"));
  rc = saf3r_pack_qkv(d, d, d, 3072, 64, 4, 1374, 5, 0, nullptr, nullptr, nullptr, nullptr, 1e-6f, 0, nullptr,
                      nullptr, nullptr, 0, d, d, d, nullptr, nullptr, nullptr, nullptr, 1.f, nullptr, nullptr, nullptr,
                      nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("num_heads"));
  rc = saf3r_pack_qkv(d, d, d, 3072, 64, 4, 1374, 5, 16, nullptr, nullptr, nullptr, nullptr, 1e-6f, 1, nullptr,
                      nullptr, nullptr, 0, d, d, d, nullptr, nullptr, nullptr, nullptr, 1.f, nullptr, nullptr, nullptr,
                      nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("LayerNorm"));
  uint8_t flags16[16] = {};
  flags16[3] = 1;
  rc = saf3r_pack_qkv(d, d, d, 3072, 64, 4, 1374, 5, 16, nullptr, nullptr, nullptr, nullptr, 1e-6f, 0, nullptr,
                      nullptr, nullptr, 0, d, d, d, nullptr, nullptr, nullptr, flags16, -1.f, nullptr, nullptr, nullptr,
                      nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("q_scale"));
  rc = saf3r_pack_qkv(d, d, d, 3072, 64, 4, 1374, 5, 16, nullptr, nullptr, nullptr, nullptr, 1e-6f, 0, nullptr,
                      nullptr, nullptr, 0, d, d, d, nullptr, nullptr, nullptr, nullptr, 1.f, flags16, nullptr, nullptr,
                      nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("pool"));

  const int32_t heads[1] = {99};
  rc = saf3r_block_pool(d, d, 4, 1374, 5, 16, heads, 1, df, df, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("out of range"));
  rc = saf3r_topk_from_scores(df, 1, 16, 4, 22, 33, di, nullptr);
  CHECK(rc == SAF3R_ERR_UNSUPPORTED && last_error_has("k must be"));
  rc = saf3r_topk_from_scores(nullptr, 1, 16, 4, 22, 4, di, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID);
  rc = saf3r_block_select(df, df, 1, 88, 4, 22, 4, 7, di, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("scope"));
  rc = saf3r_block_select(df, df, 1, 88, 4, 40, 4, 0, di, nullptr);
  CHECK(rc == SAF3R_ERR_UNSUPPORTED && last_error_has("32 blocks"));
  rc = saf3r_pooled_prepare(df, -1, dh, df, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("saf3r_pooled_prepare"));
  rc = saf3r_pooled_prepare(static_cast<float*>(fake(260)), 4, dh, df, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("aligned"));

  rc = saf3r_block_select_pooled(df, dh, df, 65536, 128, 22, 4, di, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("bad shape"));
  rc = saf3r_block_select_pooled(static_cast<float*>(fake(260)), dh, df, 7, 128, 22, 4, di, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("aligned"));
  rc = saf3r_block_select_pooled(df, dh, df, 7, 128, 22, 0, di, d, INT64_MAX, nullptr);
  CHECK(rc == SAF3R_ERR_UNSUPPORTED);
  rc = saf3r_block_select_pooled(df, dh, df, 0, 128, 22, 4, di, d, INT64_MAX, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("bad shape"));

  rc = saf3r_probe_scores(df, df, 64 * 1000, 1000, di, 1, nullptr, 0, 0.125f, nullptr, df, df, 1000, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("workspace"));
  rc = saf3r_probe_scores(df, df, 64 * 1000, 0, di, 1, nullptr, 0, 0.125f, df, df, df, 1000, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("n_tokens"));
  rc = saf3r_probe_scores(df, df, 64 * 1000, 1000, di, 1, di, 1001, 0.125f, df, df, df, 1000, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("n_samples"));
  rc = saf3r_probe_scores_noalloc(df, df, 64 * 1000, 1000, di, 65, nullptr, 0, 0.125f, df, df, 1000, nullptr);
  CHECK(rc == SAF3R_ERR_UNSUPPORTED && last_error_has("static workspace"));
  rc = saf3r_probe_scores_noalloc(nullptr, df, 64 * 1000, 1000, di, 1, nullptr, 0, 0.125f, df, df, 1000, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("null"));

  rc = saf3r_keyset_build(df, 5496, 1, di, di, di, di, 4, 1374, 5, di, 100, di, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("idx_stride"));
  rc = saf3r_keyset_build(df, 5496, 0, di, di, di, di, 4, 1374, 5, di, 5496, di, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("n_heads"));
  rc = saf3r_keyset_gather(d, 4, 1374, 5, heads, 1, d, 3072, 64, di, 5496, di, 10, d, d, 64, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("max_tiles"));

  rc = saf3r_gather_attn_fwd(&rows, &rows, &null_rows, di, 4, 10, 4, 100, 0.125f, 0, &rows, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("null"));
  rc = saf3r_gather_attn_fwd(&rows, &odd_rows, &rows, di, 4, 10, 4, 100, 0.125f, 0, &rows, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("aligned"));
  rc = saf3r_gather_attn_fwd(&rows, &rows, &rows, di, 4, 10, 4, 100, 0.125f, 0x80, &rows, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("dtype"));
  rc = saf3r_gather_attn_fwd(&rows, &rows, &rows, nullptr, 4, 10, 4, 100, 0.125f, 0, &rows, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("index list"));
  CHECK(saf3r_gather_attn_workspace_bytes(100, 512) == int64_t(100) * 8 * 66 * 4);
  CHECK(saf3r_gather_attn_workspace_bytes(-1, 512) == -1);
  CHECK(saf3r_gather_attn_workspace_bytes(10, 0) == -1);
  rc = saf3r_gather_attn_fwd_sliced(&rows, &rows, &rows, di, 4, 10, 4, 100, 0.125f, 0, &rows, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("workspace"));
  rc = saf3r_gather_attn_fwd_sliced(&rows, &rows, &rows, di, 4, 10, 4, 100, 0.125f, 0, &rows, d, 100, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("workspace"));
  rc = saf3r_gather_attn_fwd_sliced(&rows, &rows, &null_rows, di, 4, 10, 4, 100, 0.125f, 0, &rows, d, 1 << 20,
                                    nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("null"));

  rc = saf3r_token_topk(&rows, &rows, 10, 4, 1369, 0, di, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("topk"));
  rc = saf3r_token_topk(&rows, &rows, 10, 4, 1369, 200, di, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_UNSUPPORTED && last_error_has("128"));
  rc = saf3r_token_topk(&rows, &null_rows, 10, 4, 1369, 4, di, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("null"));
  rc = saf3r_token_topk(&rows, &rows, 10, 4, 1369, 64, di, d, -5, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("negative workspace"));
  rc = saf3r_token_topk(&rows, &odd_rows, 10, 4, 1369, 4, di, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("aligned"));
  rc = saf3r_token_topk(&rows, &rows, 10, 4, 1369, 64, di, nullptr, 0, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("workspace"));

  rc = saf3r_frame_topk_scores(d, 5496, 10, 4, 1369, 1, 0, 1, 4, 0, di, 100, nullptr, nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("first_stride"));
  rc = saf3r_frame_topk_scores(d, 100, 10, 4, 1369, 0, 1, 1, 4, 0, di, 100, nullptr, nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("score stride"));
  rc = saf3r_frame_topk_scores(d, 5480, 10, 4, 1370, 0, 1, 1, 4, 8, di, 100, nullptr, nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("candidate buffers"));
  rc = saf3r_frame_topk_scores(nullptr, 5480, 10, 4, 1370, 0, 1, 1, 4, 0, di, 100, nullptr, nullptr, nullptr);
  CHECK(rc == SAF3R_ERR_INVALID && last_error_has("null"));
}

// with SAF3R_FAULT_INJECT set, entries fail before looking at their arguments
static void check_fault_injection() {
  void* d = fake();
  const saf3r_rows rows = {d, 64, 0, 1 << 20, 0};
  setenv("SAF3R_FAULT_INJECT", "all", 1);
  CHECK(saf3r_token_topk(&rows, &rows, 10, 4, 1369, 4, static_cast<int32_t*>(d), nullptr, 0, nullptr) ==
        SAF3R_ERR_INJECTED);
  CHECK(last_error_has("saf3r_token_topk") && last_error_has("SAF3R_FAULT_INJECT"));
  CHECK(saf3r_block_select_pooled(nullptr, nullptr, nullptr, 0, 0, 0, 0, nullptr, nullptr, 0, nullptr) ==
        SAF3R_ERR_INJECTED);
  CHECK(saf3r_pooled_prepare(nullptr, -1, nullptr, nullptr, nullptr) == SAF3R_ERR_INJECTED);
  CHECK(saf3r_gather_attn_fwd(nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0.f, 0, nullptr, nullptr) ==
        SAF3R_ERR_INJECTED);
  CHECK(saf3r_gather_attn_fwd_sliced(nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0.f, 0, nullptr, nullptr, 0,
                                     nullptr) == SAF3R_ERR_INJECTED);
  setenv("SAF3R_FAULT_INJECT", "saf3r_keyset_build", 1);
  CHECK(saf3r_keyset_build(nullptr, 0, 0, nullptr, nullptr, nullptr, nullptr, 0, 0, 0, nullptr, 0, nullptr,
                           nullptr) == SAF3R_ERR_INJECTED);
  CHECK(saf3r_topk_from_scores(nullptr, 1, 16, 4, 22, 4, nullptr, nullptr) == SAF3R_ERR_INVALID);  // not named
  // a long entry name in the variable does not overrun the message buffer
  static char longname[2048];
  std::memset(longname, 'x', sizeof(longname) - 1);
  setenv("SAF3R_FAULT_INJECT", longname, 1);
  CHECK(saf3r_topk_from_scores(nullptr, 1, 16, 4, 22, 4, nullptr, nullptr) == SAF3R_ERR_INVALID);
  unsetenv("SAF3R_FAULT_INJECT");
}

int main() {
  check_queries();
  check_sparse_attn();
  check_other_entries();
  check_fault_injection();
  if (g_failures) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("host checks passed\n");
  return 0;
}

// C-ABI plumbing: version, thread-local last error, fault injection, layout size query.
#include "common.h"

namespace saf3r {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int injected(const char* entry) {
  const char* e = getenv("SAF3R_FAULT_INJECT");
  if (e == nullptr || e[0] == '\0') return SAF3R_OK;
  if (strcmp(e, "all") == 0 || strcmp(e, entry) == 0)
    return fail(SAF3R_ERR_INJECTED, "%s: failure injected through SAF3R_FAULT_INJECT", entry);
  return SAF3R_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SAF3R_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  set_error("");
  return SAF3R_OK;
}

}  // namespace saf3r

extern "C" int saf3r_abi_version(void) { return SAF3R_ABI_VERSION; }

extern "C" const char* saf3r_last_error(void) { return saf3r::g_last_error; }

extern "C" int64_t saf3r_packed_slots(int frames, int tokens_per_frame, int num_special) {
  saf3r::Geom g;
  if (!saf3r::make_geom(frames, tokens_per_frame, num_special, &g)) return -1;
  return g.L;
}

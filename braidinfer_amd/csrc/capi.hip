// Library-wide C ABI: version, per-thread error text and the planner overrides.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "bfa_host.h"

namespace bfa {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(BFA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return BFA_OK;
}

// Planner overrides (BFA_TUNE_* keys), -1 = unset.  Filled from the
// environment once, by the static initialiser below, when the library is
// loaded; afterwards only bfa_set_tuning writes the table.
static int g_tuning[BFA_TUNE_COUNT];

namespace {
struct TuningFromEnv {
  TuningFromEnv() {
    static const char* const names[BFA_TUNE_COUNT] = {
        "BFA_DECODE_KS",      "BFA_DECODE_WG",         "BFA_DECODE_SPLITS", "BFA_QKV_TILE",
        "BFA_EDT_RT",         "BFA_DECODE_PAIR",       "BFA_NO_OPERAND_FOLD", "BFA_CASCADE_DECODE_WG",
        "BFA_CASCADE_FLAT",   "BFA_CASCADE_FLAT_WG",   "BFA_STREAM_STORES", "BFA_QKV_PERSIST",
        "BFA_DECODE_GEMV"};
    for (int k = 0; k < BFA_TUNE_COUNT; ++k) {
      const char* v = getenv(names[k]);
      g_tuning[k] = (v != nullptr && *v != '\0') ? atoi(v) : -1;
    }
  }
};
const TuningFromEnv g_tuning_from_env;
}  // namespace

int tuning(int key) { return (key >= 0 && key < BFA_TUNE_COUNT) ? g_tuning[key] : -1; }

}  // namespace bfa

extern "C" int bfa_set_tuning(int key, int value) {
  if (key < 0 || key >= BFA_TUNE_COUNT) return bfa::set_error(BFA_ERR_INVALID, "bfa_set_tuning: unknown key %d", key);
  bfa::g_tuning[key] = value < 0 ? -1 : value;
  return BFA_OK;
}

extern "C" int bfa_get_tuning(int key) { return bfa::tuning(key); }

extern "C" int bfa_abi_version(void) { return BFA_ABI_VERSION; }

extern "C" const char* bfa_last_error(void) { return bfa::g_last_error; }

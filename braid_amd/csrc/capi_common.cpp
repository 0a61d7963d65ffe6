// Error reporting and slot validation for the C ABI (host code only).
#include "capi_common.h"

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstdlib>
#include <vector>

namespace braid {

namespace {
thread_local std::string g_last_error;
}  // namespace

int parse_knob(const char* e) {
  if (e == nullptr || e[0] == '\0') return -1;
  errno = 0;
  char* end = nullptr;
  const long v = std::strtol(e, &end, 10);
  if (errno != 0 || end == e || *end != '\0' || v < 0 || v > (1L << 30)) return -1;
  return (int)v;
}

namespace {

constexpr int kKnobs = 6;
const char* const kKnobEnv[kKnobs] = {"BRAID_DECODE_XCD_REMAP", "BRAID_DECODE_WGS_PER_CU",
                                      "BRAID_PREFILL_COLS", "BRAID_DECODE_PARTS",
                                      "BRAID_PREFILL_PLAN", "BRAID_FP8_GEMM"};

// Read once, at library load (static initialisation), not per launch. A value
// that is not a whole decimal number in [0, 2^30], or is empty, leaves the
// knob unset (-1), so a typo cannot force a launch shape.
struct Knobs {
  std::atomic<int> v[kKnobs];
  Knobs() {
    for (int i = 0; i < kKnobs; ++i)
      v[i].store(parse_knob(std::getenv(kKnobEnv[i])), std::memory_order_relaxed);
  }
};
Knobs g_knobs;
}  // namespace

int launch_knob(int knob) {
  return knob >= 0 && knob < kKnobs ? g_knobs.v[knob].load(std::memory_order_relaxed) : -1;
}

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int ok() {
  g_last_error.clear();
  return BRAID_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return BRAID_OK;
  return fail(BRAID_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool stream_capturing(hipStream_t stream, int* status) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  *status = hip_status(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
  return cs != hipStreamCaptureStatusNone;
}

namespace {
// Pinned host memory for the eager checks' small device-to-host copies, per
// thread, grown on demand: a copy into pageable memory is staged through a
// driver buffer and costs more. Never freed (no destructor), so nothing runs
// against the HIP runtime while the process exits; a thread that made an
// eager call keeps its buffer (1 KiB for up to 128 rows with lengths).
struct Staging {
  int32_t* p = nullptr;
  size_t cap = 0;
};
thread_local Staging g_staging;

int32_t* staging(size_t count, int* status) {
  if (count > g_staging.cap) {
    if (g_staging.p != nullptr) (void)hipHostFree(g_staging.p);
    g_staging.p = nullptr;
    g_staging.cap = 0;
    size_t cap = 256;
    while (cap < count) cap *= 2;
    void* p = nullptr;
    *status = hip_status(hipHostMalloc(&p, cap * sizeof(int32_t), hipHostMallocDefault),
                         "allocating pinned host memory for the slot check");
    if (*status != BRAID_OK) return nullptr;
    g_staging.p = static_cast<int32_t*>(p);
    g_staging.cap = cap;
  }
  *status = BRAID_OK;
  return g_staging.p;
}
}  // namespace

int validate_slots(const int32_t* slot_idx, int B, int64_t n_slots, bool distinct,
                   hipStream_t stream, const int32_t* lens_dev, int32_t* lens_host) {
  int st = BRAID_OK;
  if (stream_capturing(stream, &st)) return BRAID_OK;
  if (st != BRAID_OK) return st;
  if (B == 0) return BRAID_OK;
  const bool with_lens = lens_dev != nullptr && lens_host != nullptr;
  int32_t* host = staging((size_t)B * (with_lens ? 2 : 1), &st);
  if (st != BRAID_OK) return st;
  if (with_lens) {
    st = hip_status(hipMemcpyAsync(host + B, lens_dev, sizeof(int32_t) * (size_t)B,
                                   hipMemcpyDeviceToHost, stream),
                    "copying seq_lens to the host");
    if (st != BRAID_OK) return st;
  }
  st = hip_status(hipMemcpyAsync(host, slot_idx, sizeof(int32_t) * (size_t)B,
                                 hipMemcpyDeviceToHost, stream),
                  "copying slot_idx to the host");
  if (st != BRAID_OK) return st;
  st = hip_status(hipStreamSynchronize(stream), "synchronizing for slot validation");
  if (st != BRAID_OK) return st;
  if (with_lens) std::copy(host + B, host + 2 * (size_t)B, lens_host);
  std::vector<char> seen(distinct ? (size_t)n_slots : 0, 0);
  for (int i = 0; i < B; ++i) {
    const int32_t s = host[i];
    if (s < 0 || s >= n_slots) {
      return fail(BRAID_ESLOT, "slot_idx[" + std::to_string(i) + "] = " + std::to_string(s) +
                                   " is out of range [0, " + std::to_string(n_slots) + ")");
    }
    if (distinct) {
      if (seen[s]) {
        return fail(BRAID_ESLOT,
                    "slot_idx has duplicate slot " + std::to_string(s) +
                        "; two live rows sharing one state slab is silent "
                        "cross-sequence corruption. Slots must be distinct.");
      }
      seen[s] = 1;
    }
  }
  return BRAID_OK;
}

}  // namespace braid

extern "C" {

int braid_abi_version(void) { return 1; }

const char* braid_last_error(void) { return braid::g_last_error.c_str(); }

int braid_set_launch_override(int knob, int value) {
  if (knob < 0 || knob >= braid::kKnobs)
    return braid::fail(BRAID_EINVAL, "unknown launch knob " + std::to_string(knob));
  braid::g_knobs.v[knob].store(value < 0 ? -1 : value, std::memory_order_relaxed);
  return braid::ok();
}

int braid_get_launch_override(int knob) { return braid::launch_knob(knob); }

}  // extern "C"

// Error reporting and slot validation for the C ABI (host code only).
#include "capi_common.h"

#include <vector>

namespace braid {

namespace {
thread_local std::string g_last_error;
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

int validate_slots(const int32_t* slot_idx, int B, int64_t n_slots, bool distinct,
                   hipStream_t stream) {
  int st = BRAID_OK;
  if (stream_capturing(stream, &st)) return BRAID_OK;
  if (st != BRAID_OK) return st;
  if (B == 0) return BRAID_OK;
  std::vector<int32_t> host(B);
  st = hip_status(hipMemcpyAsync(host.data(), slot_idx, sizeof(int32_t) * (size_t)B,
                                 hipMemcpyDeviceToHost, stream),
                  "copying slot_idx to the host");
  if (st != BRAID_OK) return st;
  st = hip_status(hipStreamSynchronize(stream), "synchronizing for slot validation");
  if (st != BRAID_OK) return st;
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

}  // extern "C"

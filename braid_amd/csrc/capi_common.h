// Host-side helpers shared by the C-ABI entry points: thread-local error text,
// HIP status checks and the slot-map validation every pool entry performs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/braid_gdn.h"

namespace braid {

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Clears the last error and returns BRAID_OK.
int ok();

// HIP call wrapper: on failure records "<what>: <hip error string>".
int hip_status(hipError_t e, const char* what);

// True when `stream` is capturing a graph (then no host round trip is legal).
// Returns a braid status through `status`.
bool stream_capturing(hipStream_t stream, int* status);

// Copies slot_idx[0..B) to the host (skipped while capturing) and checks every
// entry lies in [0, n_slots); with `distinct`, also that no slot repeats.
// Message fragments follow braid/kernels/csrc/gdn_decode.cu:289-296:
// "... is out of range [0, n)" and "duplicate slot ... must be distinct".
// With lens_dev and lens_host, the same round trip also copies
// lens_dev[0..B) into lens_host (left untouched while capturing).
int validate_slots(const int32_t* slot_idx, int B, int64_t n_slots, bool distinct,
                   hipStream_t stream, const int32_t* lens_dev = nullptr,
                   int32_t* lens_host = nullptr);

// Launch knobs, for measurement: overrides of the launch-shape choices,
// -1 when unset. Initialised once from the environment when the library
// loads (BRAID_DECODE_XCD_REMAP, BRAID_DECODE_WGS_PER_CU, BRAID_PREFILL_COLS,
// BRAID_DECODE_PARTS, BRAID_PREFILL_PLAN, BRAID_FP8_GEMM), then changed only by
// braid_set_launch_override. The knobs are process-wide: an override set on
// one thread shapes the launches of every thread.
int launch_knob(int knob);

// A knob's value from its environment string: a whole decimal number in
// [0, 2^30], else -1 (unset): empty, non-numeric, trailing text, negative.
int parse_knob(const char* e);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace braid

// Host-side helpers shared by the C-ABI entry points: error state and argument checks.
#pragma once

#include <stdint.h>

#include "../../include/mamba3_hip.h"

namespace m3 {

// Record a failure for m3_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline bool present(const m3_tensor& t) { return t.ptr != nullptr; }

inline bool valid_dtype(int d) { return d == M3_F32 || d == M3_BF16 || d == M3_F16; }

inline int elem_size(int d) { return d == M3_F32 ? 4 : 2; }

// Check a required or optional tensor: dtype in range, innermost stride 1 (when `dims` > 0 and
// the innermost extent is > 1), alignment of the base pointer to its element size.
int check_tensor(const m3_tensor& t, const char* name, int dims, int64_t inner_extent,
                 bool required, int want_dtype /* -1: any */);

// After a launch: translate hipGetLastError into a status.
int check_launch(const char* what);

// The recurrent scan (rscan.hip) for the shapes the chunked MFMA kernel does not tile, and a
// decode step run as a one-token recurrent scan for the shapes the step kernels do not take.
bool rscan_fits(const m3_scan_args& a);
int launch_recurrent_scan(const m3_scan_args& a, hipStream_t stream);
m3_scan_args step_as_scan(const m3_step_args& s);
int launch_recurrent_step(const m3_step_args& s, hipStream_t stream);

}  // namespace m3

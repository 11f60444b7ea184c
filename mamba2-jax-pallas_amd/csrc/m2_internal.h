// Internal launchers shared by the per-stage entry points and m2_ssd_combined.
// Each validates its arguments, enqueues its kernel(s) on `stream` and returns
// an M2_* code (the message goes to m2_last_error).
#pragma once

#include "m2_common.h"

namespace m2 {
int launch_chunk_cumsum(const m2_chunk_cumsum_args& a, hipStream_t stream);
int launch_chunk_state(const m2_chunk_state_args& a, hipStream_t stream);
int launch_state_passing(const m2_state_passing_args& a, hipStream_t stream);
int launch_bmm_chunk(const m2_bmm_chunk_args& a, hipStream_t stream);
int launch_chunk_scan(const m2_chunk_scan_args& a, hipStream_t stream);
int launch_chunk_state_varlen(const m2_chunk_state_varlen_args& a, hipStream_t stream);
int launch_ssu(const m2_ssu_args& a, hipStream_t stream);
}  // namespace m2

// Library-internal SpGEMM interface shared by the symbolic phase
// (spgemm_symbolic.hip) and the A-stationary numeric phase (spgemm_astat.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "diagpu.h"

namespace diagpu {

// Queues on `s` the records of diagpu_spgemm_astat_prepare for the plan the
// multi-launch symbolic phase queued before it on `s` is building: records[4 g .. 4 g + 3]
// for every entry g and, after them, {0, 0, smallest, largest A offset}.
// The plan's counts are read on the device from that phase's state record
// (state_counts[0] C diagonals, [2] entries, bounded by c_capacity and
// pair_capacity); nothing is written if its flags (state_flags[0]) are
// non-zero, and the step ORs its own errors into state_flags[1] (1: an entry
// not in the symbolic form, 2: a B index beyond 2^30 - 1).  c_bound: an upper
// bound of the C diagonal count known on the host (sizes the grid).  records
// holds 4 pair_capacity + 4 int32.  Asynchronous.
int launch_astat_records(hipStream_t s, int32_t n, const int32_t* A_off,
                         const int64_t* A_starts, int32_t nA, const int32_t* B_off,
                         const int64_t* B_starts, int32_t nB, const int32_t* C_off,
                         const int64_t* pair_ptr, int64_t c_bound, int64_t c_capacity,
                         const diagpu_gpair* pairs, int64_t pair_capacity,
                         const int64_t* state_counts, int32_t* state_flags, int32_t* records);

}  // namespace diagpu

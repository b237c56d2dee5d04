// Internal interface between the C ABI (dz_api.hip) and the kernels (dz_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dz_common.h"

namespace dz {

enum RmwMode : int { kModePerturb = 0, kModeUpdate = 1, kModeRestoreUpdate = 2 };
enum ProjMode : int { kProjSumsq = 0, kProjApply = 1, kProjReverse = 2, kProjReverseSumsq = 3 };

// Read-modify-write kernel geometry. A workgroup of 1024 threads takes one
// tile (chunk) at a time from the table's work counters; each thread owns
// kRmwGroups16 (16-bit T) or kRmwGroups32 (fp32) groups of 8 elements per
// tile, i.e. 128 KB of theta per tile for every dtype.
constexpr int kRmwThreads = 1024;
constexpr int kRmwGroups16 = 8;
constexpr int kRmwGroups32 = 4;
constexpr int kRmwChunk16 = kRmwThreads * kRmwGroups16 * 8;  // 65536 elements
constexpr int kRmwChunk32 = kRmwThreads * kRmwGroups32 * 8;  // 32768 elements
__host__ __device__ constexpr int rmw_chunk_elems(int dtype) {
  return dtype == DZ_F32 ? kRmwChunk32 : kRmwChunk16;
}

// LDS bytes of the per-launch delta table of an RMW launch: 16-bit entries
// for perturb/update of 16-bit T, 32-bit entries otherwise (fp32 deltas, or
// the (restore delta, update delta) pair of a fused restore+update).
__host__ __device__ constexpr int rmw_lds_table_bytes(int dtype, int mode) {
  return (dtype == DZ_F32 || mode == kModeRestoreUpdate) ? kDzTabEntries * 4 : kDzTabEntries * 2;
}

// Work counters of a table, one set per table: kCounters tile dispensers 128
// bytes apart, then the number of finished workgroups. Zeroed when the table
// is created; the last workgroup of every RMW launch puts them back to zero,
// so consecutive launches on one stream need no reset (and no memset in a
// captured graph). Launches of one table must not overlap in time.
constexpr int kCounters = 8;
constexpr int kCounterStride = 32;  // uint32 slots (128 bytes)
constexpr int kCounterWords = (kCounters + 1) * kCounterStride;

// Projection kernel geometry: 256 threads x 32 elements (16-bit T: 4 x 16 B,
// fp32: 8 x 16 B per thread).
constexpr int kProjThreads = 256;
constexpr int kProjChunk = 8192;

// By-value scalars of one RMW launch.
struct DzScalars {
  uint64_t seed;
  float scale;  // scaling_factor s of the perturbation
  float eps;    // zo_eps
  float grad;   // projected_grad g
  float lr;     // learning rate of this update
};

// Optional device-resident overrides (read by the kernel when non-null), so a
// captured graph can replay with a new seed / gradient / learning rate.
struct DzScalarPtrs {
  const uint64_t* seed;  // device uint64
  const void* grad;      // device scalar of the table dtype T
  const float* lr;       // device fp32
};

hipError_t launch_rmw(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t grid,
                      const void* qtab, const DzScalars& s, const DzScalarPtrs& p, uint32_t* counters,
                      hipStream_t st);
hipError_t launch_proj(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, const void* alpha,
                       double* partials, hipStream_t st);
hipError_t launch_finalize(int dtype, const double* partials, const uint32_t* gbegin, uint32_t ngroups,
                           double* sumsq, float* norm_f32, void* norm_T, hipStream_t st);
hipError_t launch_normals(int dtype, const void* tab, uint64_t seed, uint32_t stream, uint64_t offset,
                          uint64_t n, void* out, hipStream_t st);
hipError_t launch_philox(uint64_t seed, uint32_t stream, uint64_t q0, uint64_t n, uint32_t* out,
                         hipStream_t st);

}  // namespace dz

// Internal interface between the C ABI (dz_api.hip) and the kernels (dz_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dz_common.h"

namespace dz {

// Read-modify-write kernel geometry: 1024 threads x 4 groups x 8 elements.
constexpr int kRmwThreads = 1024;
constexpr int kUnroll = 4;
constexpr int kRmwChunk = kRmwThreads * kUnroll * 8;  // 32768 elements

// Projection kernel geometry: 256 threads x 32 elements (16-bit T: 4 x 16 B,
// fp32: 8 x 16 B per thread).
constexpr int kProjThreads = 256;
constexpr int kProjChunk = 8192;

enum RmwMode : int { kModePerturb = 0, kModeUpdate = 1, kModeRestoreUpdate = 2 };
enum ProjMode : int { kProjSumsq = 0, kProjApply = 1, kProjReverse = 2, kProjReverseSumsq = 3 };

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
                      const void* tab, const DzScalars& s, const DzScalarPtrs& p, hipStream_t st);
hipError_t launch_proj(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, const void* alpha,
                       double* partials, hipStream_t st);
hipError_t launch_finalize(int dtype, const double* partials, const uint32_t* gbegin, uint32_t ngroups,
                           double* sumsq, float* norm_f32, void* norm_T, hipStream_t st);
hipError_t launch_normals(int dtype, const void* tab, uint64_t seed, uint32_t stream, uint64_t offset,
                          uint64_t n, void* out, hipStream_t st);
hipError_t launch_philox(uint64_t seed, uint32_t stream, uint64_t q0, uint64_t n, uint32_t* out,
                         hipStream_t st);

}  // namespace dz

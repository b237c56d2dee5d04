// Internal interface between the C ABI (dz_api.hip) and the kernels (dz_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dz_common.h"

namespace dz {

enum RmwMode : int {
  kModePerturb = 0,               // theta + b(z)
  kModeUpdate = 1,                // theta - d(z)
  kModeRestoreUpdate = 2,         // theta + b(z) - d(z)
  kModeRestoreUpdatePerturb = 3,  // theta + b(z) - d(z) + b(z'), z' from a second seed
};
// Modes whose table entries hold the pair (b, -d).
__host__ __device__ constexpr bool rmw_pair_mode(int mode) {
  return mode == kModeRestoreUpdate || mode == kModeRestoreUpdatePerturb;
}
enum ProjMode : int {
  kProjSumsq = 0,         // per-chunk sums of R_T(theta - theta0)^2
  kProjApply = 1,         // theta <- R(R(R(theta - theta0) * alpha) + theta0), alpha in T
  kProjReverse = 2,       // theta <- R(R(R(theta - theta0) / alpha) + theta0)
  kProjReverseSumsq = 3,  // REVERSE, then the sums of the new theta
  kProjApplyF32 = 4,      // theta <- R_T(fp32(R(theta - theta0)) * alpha + theta0), alpha fp32
};
// Most groups one dot launch takes (their pointers travel as kernel
// arguments); dz_group_dot launches once per batch of groups.
constexpr int kMaxDotGroups = 128;
struct DzPtrArray {
  uint64_t p[kMaxDotGroups];
};

// Read-modify-write kernel geometry. A workgroup of 1024 threads takes one
// tile at a time from the table's work counters; each thread owns
// rmw_groups(dtype, mode) groups of 8 elements per tile. Measured on the MI355X at
// OPT-13B size (643 tensors, fp16): 64 KB tiles (four groups per thread) and
// one workgroup per CU stream best for every mode: perturb 6.4 TB/s against
// 6.05 with 16 KB tiles and two workgroups per CU (which a 64 KB table would
// allow); 32 KB and 128 KB tiles were no better, and the three-way pass took
// 7.96 ms with six groups per thread and spilled with eight. fp32 uses 32 KB
// tiles (one group of 8 fp32 per thread): its only workload, OPT-125m (347 MB
// of parameters, about 40 tiles per CU), runs a pass in 121 us that way
// against 140 us with 64 KB tiles. The bf16 restore + update + next
// perturbation pass (prefetching loop, ALU-bound) takes three groups per
// thread (48 KB tiles): at OPT-30B 18.87-18.94 ms against 19.79-19.86 ms with
// four and 19.57-19.62 with two (same box, alternating builds), where the
// single-value bf16 passes take 19.3 ms with three and 17.6 with four, and
// the fp16 three-way pass 8.07 ms with three against 7.60 with four. A table
// whose three-way tile size differs keeps a second tile list for it.
constexpr int kRmwThreads = 1024;
__host__ __device__ constexpr int rmw_groups(int dtype, int mode) {
  return dtype == DZ_F32 ? 1 : (dtype == DZ_BF16 && mode == kModeRestoreUpdatePerturb) ? 3 : 4;
}
// Elements per tile of an RMW launch (the size of the table's tile list it runs over).
__host__ __device__ constexpr int rmw_chunk_elems(int dtype, int mode) {
  return kRmwThreads * rmw_groups(dtype, mode) * 8;
}

// LDS bytes of the per-launch delta table of an RMW launch: 16-bit entries
// for perturb/update of 16-bit T, 32-bit entries otherwise (fp32 deltas, or
// the (restore delta, update delta) pair of a fused restore+update).
__host__ __device__ constexpr int rmw_lds_table_bytes(int dtype, int mode) {
  return (dtype == DZ_F32 || rmw_pair_mode(mode)) ? kDzTabEntries * 4 : kDzTabEntries * 2;
}

// Work counters of a table, one set per table, 128 bytes apart: kCounters
// tile (chunk) dispensers, then (slot kDoneSlot) the number of finished
// workgroups. Zeroed when the table is created; the last workgroup of every
// launch puts them back to zero, so consecutive launches on one stream need
// no reset (and no memset in a captured graph). Launches of one table must
// not overlap in time. Four counters stream as fast as eight at OPT-13B
// (every mode within 0.3 %), sixteen 0.6-1.2 % slower; a single counter
// serialises at about 11 ns per atomic.
constexpr int kCounters = 8;
constexpr int kDoneSlot = kCounters;
constexpr int kCounterStride = 32;  // uint32 slots (128 bytes)
constexpr int kCounterWords = (kDoneSlot + 1) * kCounterStride;

// Tile loops of the RMW launches. The restore + update + next perturbation
// passes, whose ALU work per tile is the largest, run the prefetching loop
// (rmw_tiles_prefetch: the next full tile's loads go out once the tile's
// first group is stored; with fp32's one group per thread, before the tile's
// Philox chain). Measured on the MI355X, same box, alternating builds, kernel
// microbench: OPT-13B fp16 7.86-7.90 -> 7.58-7.61 ms, OPT-30B bf16
// 20.10-20.16 -> 19.83-19.95 ms, OPT-125m fp32 0.1220-0.1227 -> 0.1205-0.1207
// ms (in the step 0.1216-0.1217 -> 0.1210-0.1211; with the loads issued after
// the tile's store instead, 0.130 ms). The single-Philox passes run the same
// on either loop (OPT-13B fp16 perturb 7.66-7.69 ms both, OPT-30B bf16
// 17.76 ms both) and keep the plain loop (rmw_tiles).
__host__ __device__ constexpr bool rmw_prefetch_mode(int dtype, int mode) {
  return mode == kModeRestoreUpdatePerturb;
}
// A table's default for the launches that use the prefetching loop: those of
// at least this many tiles (dz_table_set_prefetch_min_tiles sets it per
// table). 0: every launch of such a mode. With the next tile's loads issued
// inside the tile's work, the prefetching loop is also the faster one for a short pass
// (OPT-2.7B fp16, 77 K tiles, in the ZO step: 1.544-1.545 against
// 1.562-1.563 ms).
constexpr uint32_t kPrefetchMinTilesDefault = 0;

// Projection kernel geometry: persistent 1024-thread workgroups, one per CU,
// taking chunks of proj_chunk_elems(dtype) elements: 32768 for 16-bit T (64 KB
// of theta and 64 KB of theta0, 4 16-byte vectors of each per thread), 8192
// for fp32 (32 KB, 2 vectors). Two workgroups per CU streamed slower (6.49
// against 6.76 TB/s for a bare two-read-one-write kernel), as did smaller
// workgroups on one counter. fp32's only workload, OPT-125m, projects 57 MB
// per stream: 432 chunks of 32768 left two thirds of the CUs with two chunks
// and the rest with one. In its ZO step (same box, two alternating runs
// each), apply / norm / reverse+norm took 46 / 36 / 47 us with 32768-element
// chunks, 34 / 30 / 40 with 16384, 32 / 31 / 40 with 8192 and 31 / 37 / 44
// with 4096.
constexpr int kProjThreads = 1024;
__host__ __device__ constexpr int proj_chunk_elems(int dtype) { return dtype == DZ_F32 ? 8192 : 32768; }
// Groups whose alphas a projection workgroup keeps in LDS (16 KB of fp32);
// beyond that each chunk reads its group's alpha from memory.
constexpr int kProjAlphaLds = 4096;

// By-value scalars of one RMW launch.
struct DzScalars {
  uint64_t seed;
  uint64_t seed2;  // seed of the next step's perturbation (kModeRestoreUpdatePerturb)
  float scale;  // scaling_factor s of the perturbation
  float eps;    // zo_eps
  float grad;   // projected_grad g
  float lr;     // learning rate of this update
};

// Optional device-resident overrides (read by the kernel when non-null), so a
// captured graph can replay with a new seed / gradient / learning rate.
struct DzScalarPtrs {
  const uint64_t* seed;   // device uint64
  const uint64_t* seed2;  // device uint64
  const void* grad;      // device scalar of the table dtype T
  const float* lr;       // device fp32
};

// Timing events of one launch: when set, the runtime records `start` as the
// kernel starts and `stop` as it ends (hipExtLaunchKernel), so an event pair
// brackets the kernel itself rather than the host's launch work as well.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

// The chunk list holds its full, aligned tiles first; the rest are partial
// or misaligned. prefetch: run the prefetching tile loop where the mode
// allows it (rmw_prefetch_mode); the caller sets it for long launches.
hipError_t launch_rmw(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t grid,
                      const void* qtab, const DzScalars& s, const DzScalarPtrs& p, uint32_t* counters,
                      bool prefetch, hipStream_t st, const LaunchEvents& ev = {});
// Persistent: `grid` workgroups share the chunks through `counters` (zero
// before the launch; the launch leaves them at zero).
hipError_t launch_proj(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t ngroups,
                       uint32_t grid, const void* alpha, double* partials, uint32_t* counters, hipStream_t st,
                       const LaunchEvents& ev = {});
// Chunks of groups group_base .. group_base + kMaxDotGroups - 1; other.p[i]
// is the tensor of group group_base + i.
hipError_t launch_dot(int dtype, const DzChunk* chunks, uint32_t nchunks, const DzPtrArray& other,
                      uint32_t group_base, double* partials, hipStream_t st, const LaunchEvents& ev = {});
// take_sqrt: norms (sqrt of the sums) or plain sums in the fp32 / T outputs.
hipError_t launch_finalize(int dtype, const double* partials, const uint32_t* gbegin, uint32_t ngroups,
                           double* sumsq, float* norm_f32, void* norm_T, bool take_sqrt, hipStream_t st,
                           const LaunchEvents& ev = {});
// Chunk plan of a projection launch without a table (dz_group_sumsq_static):
// kStaticPlanGroups groups per plan launch, their descriptors and the
// group -> chunk index written into caller-provided device memory.
constexpr int kStaticPlanGroups = 64;
struct StaticPlanBatch {
  uint64_t ptr[kStaticPlanGroups];
  uint64_t anchor[kStaticPlanGroups];
  int64_t numel[kStaticPlanGroups];
  uint32_t chunk_begin[kStaticPlanGroups];  // first chunk of each group of the batch
  uint32_t ngroups;                         // groups in this batch
  uint32_t group_base;                      // index of the batch's first group
  uint32_t total_groups;
  uint32_t total_chunks;
  int32_t elem_size;
  int32_t chunk_elems;  // proj_chunk_elems(dtype)
  uint32_t first;       // the first batch also zeroes the work counters
};
hipError_t launch_static_plan(const StaticPlanBatch& b, DzChunk* chunks, uint32_t* group_begin, uint32_t* counters,
                              hipStream_t st);
hipError_t launch_normals(int dtype, const void* tab, uint64_t seed, uint32_t stream, uint64_t offset,
                          uint64_t n, void* out, hipStream_t st);
hipError_t launch_philox(uint64_t seed, uint32_t stream, uint64_t q0, uint64_t n, uint32_t* out,
                         hipStream_t st);

}  // namespace dz

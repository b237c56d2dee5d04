// C ABI of the DiZO ZO-step library (declared in include/dizo_amd.h).
//
// Responsibilities: argument validation, the host-side chunk lists of each
// parameter table, per-device quantile tables, and error reporting. Every
// kernel launch is preceded by checks that the table belongs to the current
// device and that all registered ranges lie inside their allocations.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/dizo_amd.h"
#include "dz_common.h"
#include "dz_kernels.h"

namespace {

thread_local std::string g_last_error;

int32_t fail(int32_t code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int32_t hip_fail(hipError_t e, const char* what) {
  return fail(DZ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int elem_size(int32_t dtype) { return dtype == DZ_DTYPE_F32 ? 4 : 2; }

bool valid_dtype(int32_t dtype) {
  return dtype == DZ_DTYPE_F32 || dtype == DZ_DTYPE_F16 || dtype == DZ_DTYPE_BF16;
}

// ---------------------------------------------------------------------------
// Quantile table: Q[i] = RNE_T(Phi^{-1}(1/2 + (i + 1/2)/65536)), i < 32768.
// ---------------------------------------------------------------------------

// x > 0 with Phi(x) = 1/2 + r, 0 < r < 1/2, to about one double ulp. Newton
// iterations on the well-conditioned form of Phi(x) - 1/2 - r: 0.5*erf(x/sqrt2) - r
// near the centre, (1/2 - r) - 0.5*erfc(x/sqrt2) in the tail.
double inv_normal_half(double r) {
  const double q = 0.5 - r;
  double x;
  if (r < 0.25) {
    x = r * 2.5066282746310002;  // r * sqrt(2 pi): Phi'(0) = 1/sqrt(2 pi)
  } else {
    // Abramowitz & Stegun 26.2.23 rational approximation (|error| < 4.5e-4).
    const double t = sqrt(-2.0 * log(q));
    x = t - (2.515517 + t * (0.802853 + t * 0.010328)) /
                (1.0 + t * (1.432788 + t * (0.189269 + t * 0.001308)));
  }
  for (int it = 0; it < 12; ++it) {
    const double g = (r < 0.25) ? 0.5 * erf(x * M_SQRT1_2) - r : q - 0.5 * erfc(x * M_SQRT1_2);
    const double phi = exp(-0.5 * x * x) * 0.39894228040143267794;  // 1/sqrt(2 pi)
    const double dx = g / phi;
    x -= dx;
    if (fabs(dx) <= 1e-17 * x) break;
  }
  return x;
}

// Round a positive finite double to a binary format with p significand bits
// and minimum normal exponent emin (round to nearest, ties to even).
double round_format(double x, int p, int emin) {
  int e2;
  frexp(x, &e2);  // x = m * 2^e2, m in [0.5, 1)
  int E = e2 - 1;
  if (E < emin) E = emin;
  const double quantum = ldexp(1.0, E - (p - 1));
  return nearbyint(x / quantum) * quantum;
}

uint16_t f16_bits_of_exact(double v) {  // v > 0, exactly representable in fp16
  if (v < ldexp(1.0, -14)) return (uint16_t)(v / ldexp(1.0, -24));
  int e2;
  frexp(v, &e2);
  const int E = e2 - 1;
  const uint32_t mant = (uint32_t)(v / ldexp(1.0, E - 10)) - 1024u;
  return (uint16_t)(((uint32_t)(E + 15) << 10) | mant);
}

struct HostTables {
  uint32_t f32[kDzTabEntries];
  uint16_t f16[kDzTabEntries];
  uint16_t bf16[kDzTabEntries];
};

const HostTables& host_tables() {
  static HostTables t;
  static std::once_flag once;
  std::call_once(once, [] {
    for (int i = 0; i < kDzTabEntries; ++i) {
      const double r = ((double)i + 0.5) / 65536.0;
      const double x = inv_normal_half(r);
      const float f32 = (float)round_format(x, 24, -126);
      uint32_t u;
      memcpy(&u, &f32, 4);
      t.f32[i] = u;
      t.f16[i] = f16_bits_of_exact(round_format(x, 11, -14));
      const float bf = (float)round_format(x, 8, -126);
      memcpy(&u, &bf, 4);
      t.bf16[i] = (uint16_t)(u >> 16);
    }
  });
  return t;
}

const void* host_table_ptr(int32_t dtype) {
  const HostTables& t = host_tables();
  if (dtype == DZ_DTYPE_F32) return t.f32;
  if (dtype == DZ_DTYPE_F16) return t.f16;
  return t.bf16;
}

// ---------------------------------------------------------------------------
// Per-device state: quantile tables in device memory and the CU count.
// ---------------------------------------------------------------------------
constexpr int kMaxDevices = 64;

struct DeviceState {
  bool ready = false;
  void* tab[3] = {nullptr, nullptr, nullptr};
  int cus = 0;
};

std::mutex g_dev_mu;
DeviceState g_dev[kMaxDevices];

int32_t current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (*dev < 0 || *dev >= kMaxDevices) return fail(DZ_ERR_DEVICE, "device index out of range");
  return DZ_OK;
}

// Must be called with `dev` current.
int32_t ensure_device(int dev, DeviceState** out) {
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DeviceState& s = g_dev[dev];
  if (!s.ready) {
    hipError_t e = hipDeviceGetAttribute(&s.cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(MultiprocessorCount)");
    for (int d = 0; d < 3 && e == hipSuccess; ++d) {
      const size_t bytes = (size_t)kDzTabEntries * (size_t)elem_size(d);
      e = hipMalloc(&s.tab[d], bytes);
      if (e == hipSuccess) e = hipMemcpy(s.tab[d], host_table_ptr(d), bytes, hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
      // leave the state as it was, so that a later call starts over
      for (void*& p : s.tab) {
        if (p) (void)hipFree(p);
        p = nullptr;
      }
      return hip_fail(e, "quantile table upload");
    }
    s.ready = true;
  }
  *out = &s;
  return DZ_OK;
}

// Checks [p, p + bytes) lies inside one device allocation.
int32_t check_range(uint64_t p, uint64_t bytes, const char* what, int32_t i) {
  if (p == 0) return fail(DZ_ERR_INVALID, std::string(what) + " pointer is NULL (tensor " + std::to_string(i) + ")");
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  hipError_t e = hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)(uintptr_t)p);
  if (e != hipSuccess) {
    return fail(DZ_ERR_RANGE, std::string(what) + " of tensor " + std::to_string(i) +
                                  " is not device memory: " + hipGetErrorString(e));
  }
  const uint64_t b = (uint64_t)(uintptr_t)base;
  if (p < b || p + bytes > b + (uint64_t)size) {
    return fail(DZ_ERR_RANGE, std::string(what) + " range of tensor " + std::to_string(i) +
                                  " exceeds its allocation");
  }
  return DZ_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (dz_group_sumsq_static): device
// memory the library never allocates at run time. Layout: the projection
// kernel's work counters, the group -> first chunk index, the chunk
// descriptors and the per-chunk partial sums, for at most kStaticMaxGroups
// groups and kStaticMaxChunks chunks of proj_chunk_elems(dtype) elements (8.6 G
// elements of a 16-bit type, 2.1 G of fp32).
// Each device holds its own copy, at its own address (see static_scratch).
// ---------------------------------------------------------------------------
namespace {
constexpr uint32_t kStaticMaxGroups = 4096;
constexpr uint32_t kStaticMaxChunks = 1u << 18;
constexpr size_t kStaticOffCounters = 0;
constexpr size_t kStaticOffGroupBegin = 4096;
constexpr size_t kStaticOffChunks = kStaticOffGroupBegin + ((kStaticMaxGroups + 1) * 4 + 255) / 256 * 256;
constexpr size_t kStaticOffPartials = kStaticOffChunks + (size_t)kStaticMaxChunks * sizeof(DzChunk);
constexpr size_t kStaticBytes = kStaticOffPartials + (size_t)kStaticMaxChunks * sizeof(double);
static_assert(dz::kCounterWords * 4 <= kStaticOffGroupBegin, "work counters overflow their scratch slot");
}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

struct dz_table {
  int device = -1;
  int32_t dtype = 0;
  bool projection = false;
  int32_t n = 0;
  uint32_t chunk_elems = 0;  // tile size (elements)
  uint32_t nchunks = 0;      // ZO tables: full, aligned tiles first (the prefetching loop runs them)
  std::vector<uint64_t> ptrs, aux, zoff;
  std::vector<int64_t> numels;
  std::vector<uint32_t> group_begin;  // n + 1 chunk indices (projection tables)
  DzChunk* d_chunks = nullptr;
  // ZO tables whose restore + update + next perturbation launches use another
  // tile size (rmw_chunk_elems): their own tile list, else empty
  uint32_t fused_elems = 0;
  uint32_t fused_nchunks = 0;
  DzChunk* d_fused_chunks = nullptr;
  uint32_t* d_group_begin = nullptr;
  double* d_partials = nullptr;
  uint32_t* d_counters = nullptr;  // work counters of the persistent RMW / projection kernels
  DeviceState* dev = nullptr;
  dz::LaunchEvents timing;  // dz_table_time_next's request for the next launching call
  // launches of at least this many tiles run the prefetching tile loop (where
  // the mode allows it; dz_table_set_prefetch_min_tiles)
  uint32_t prefetch_min_tiles = dz::kPrefetchMinTilesDefault;
};

namespace {

// The table's pending timing request, taken (and cleared) by a launching call.
dz::LaunchEvents take_timing(dz_table* t) {
  const dz::LaunchEvents ev = t->timing;
  t->timing = dz::LaunchEvents{};
  return ev;
}

// A call with nothing to launch records its timing pair back to back on the
// stream, so the pair still brackets the call's (empty) device work.
int32_t record_unlaunched(const dz::LaunchEvents& ev, void* stream) {
  for (hipEvent_t e : {ev.start, ev.stop}) {
    if (!e) continue;
    const hipError_t r = hipEventRecord(e, (hipStream_t)stream);
    if (r != hipSuccess) return hip_fail(r, "hipEventRecord (timing of a call with nothing to launch)");
  }
  return DZ_OK;
}

int32_t check_table(const dz_table* t) {
  if (!t) return fail(DZ_ERR_INVALID, "table is NULL");
  int dev;
  int32_t rc = current_device(&dev);
  if (rc) return rc;
  if (dev != t->device) {
    return fail(DZ_ERR_DEVICE, "table lives on device " + std::to_string(t->device) +
                                   " but the current device is " + std::to_string(dev));
  }
  return DZ_OK;
}

void free_table(dz_table* t) {
  if (t->d_chunks) (void)hipFree(t->d_chunks);
  if (t->d_fused_chunks) (void)hipFree(t->d_fused_chunks);
  if (t->d_group_begin) (void)hipFree(t->d_group_begin);
  if (t->d_partials) (void)hipFree(t->d_partials);
  if (t->d_counters) (void)hipFree(t->d_counters);
  delete t;
}

// Optional per-group outputs must each hold t->n values.
int32_t check_group_outputs(const dz_table* t, const double* d_sumsq, const float* d_norm_f32,
                            const void* d_norm_T) {
  int32_t rc = DZ_OK;
  if (d_sumsq) rc = check_range((uint64_t)(uintptr_t)d_sumsq, (uint64_t)t->n * 8, "sumsq", 0);
  if (!rc && d_norm_f32) rc = check_range((uint64_t)(uintptr_t)d_norm_f32, (uint64_t)t->n * 4, "norm_f32", 0);
  if (!rc && d_norm_T)
    rc = check_range((uint64_t)(uintptr_t)d_norm_T, (uint64_t)t->n * elem_size(t->dtype), "norm_T", 0);
  return rc;
}

// Persistent grid of an RMW launch: one 1024-thread workgroup per CU, but no
// more than there are tiles.
uint32_t rmw_grid(const dz_table* t, uint32_t ntiles) {
  const uint32_t g = (uint32_t)t->dev->cus;
  return ntiles < g ? ntiles : g;
}

// Persistent grid of a projection launch: one workgroup per CU, but no more
// than there are chunks.
uint32_t proj_grid(const dz_table* t) {
  const uint32_t g = (uint32_t)t->dev->cus;
  return t->nchunks < g ? t->nchunks : g;
}

int32_t rmw(dz_table* t, int mode, const dz::DzScalars& s, const dz::DzScalarPtrs& p, void* stream) {
  int32_t rc = check_table(t);
  if (rc) return rc;
  const dz::LaunchEvents ev = take_timing(t);
  if (t->projection) return fail(DZ_ERR_INVALID, "perturb/update need a ZO table (created without anchors)");
  // the tile list whose tile size the launch's kernel takes
  const uint32_t want = (uint32_t)dz::rmw_chunk_elems(t->dtype, mode);
  const DzChunk* chunks = t->d_chunks;
  uint32_t ntiles = t->nchunks;
  if (want != t->chunk_elems) {
    if (want != t->fused_elems) return fail(DZ_ERR_INVALID, "internal: no tile list for this launch");
    chunks = t->d_fused_chunks;
    ntiles = t->fused_nchunks;
  }
  if (ntiles == 0) return record_unlaunched(ev, stream);
  hipError_t e = dz::launch_rmw(t->dtype, mode, chunks, ntiles, rmw_grid(t, ntiles), t->dev->tab[t->dtype], s, p,
                                t->d_counters, ntiles >= t->prefetch_min_tiles, (hipStream_t)stream, ev);
  if (e != hipSuccess) return hip_fail(e, "rmw kernel launch");
  return DZ_OK;
}

// Tiles of `elems` elements over every registered tensor, in tensor order.
void build_chunks(const dz_table* t, uint32_t elems, std::vector<DzChunk>* out,
                  std::vector<uint32_t>* group_begin) {
  const int es = elem_size(t->dtype);
  out->clear();
  if (group_begin) group_begin->assign(1, 0u);
  for (int32_t i = 0; i < t->n; ++i) {
    const int64_t ne = t->numels[i];
    const uint64_t p = t->ptrs[i], a = t->aux[i], z = t->zoff[i];
    const bool aligned = (p % 16 == 0) && (a % 16 == 0);
    for (int64_t s = 0; s < ne; s += elems) {
      DzChunk c;
      c.ptr = p + (uint64_t)s * es;
      c.aux = t->projection ? a + (uint64_t)s * es : 0;
      c.zgroup = t->projection ? (uint64_t)s : (z + (uint64_t)s) >> 3;
      c.n = (uint32_t)((ne - s) < (int64_t)elems ? (ne - s) : elems);
      c.meta = (uint32_t)i | (aligned ? kDzMetaAligned : 0u);
      out->push_back(c);
    }
    if (group_begin) group_begin->push_back((uint32_t)out->size());
  }
}

// ZO tile lists: full, aligned tiles first (in tensor order), then the
// partial or misaligned ones; returns the number of full tiles. The order of
// the tiles changes no result (z is a function of the element index), and it
// lets the RMW kernel run its full tiles without a per-tile shape test.
uint32_t full_tiles_first(std::vector<DzChunk>* v, uint32_t elems) {
  auto it = std::stable_partition(v->begin(), v->end(), [elems](const DzChunk& c) {
    return c.n == elems && (c.meta & kDzMetaAligned) != 0u;
  });
  return (uint32_t)(it - v->begin());
}

// Rejects a table in which a range the kernels write (theta) overlaps another
// registered range: within one launch the tiles of both would be read and
// written by different workgroups in no fixed order. Anchors are only read
// and may overlap each other (one anchor shared by several groups).
int32_t check_no_overlap(const dz_table* t) {
  struct Range {
    uint64_t lo, hi;
    bool write;
    int32_t idx;
  };
  const int es = elem_size(t->dtype);
  std::vector<Range> r;
  r.reserve((size_t)t->n * (t->projection ? 2 : 1));
  for (int32_t i = 0; i < t->n; ++i) {
    if (t->numels[i] == 0) continue;
    const uint64_t bytes = (uint64_t)t->numels[i] * es;
    r.push_back({t->ptrs[i], t->ptrs[i] + bytes, true, i});
    if (t->projection) r.push_back({t->aux[i], t->aux[i] + bytes, false, i});
  }
  std::sort(r.begin(), r.end(), [](const Range& a, const Range& b) { return a.lo < b.lo; });
  // Sorted by start, a range overlaps an earlier one iff it starts below the
  // largest end seen so far (of any range, or of a written one).
  uint64_t end_any = 0, end_write = 0;
  int32_t who_any = -1, who_write = -1;
  for (const Range& x : r) {
    const bool clash = x.write ? (x.lo < end_any) : (x.lo < end_write);
    if (clash) {
      const int32_t other = x.write ? who_any : who_write;
      return fail(DZ_ERR_INVALID, "the memory of tensor " + std::to_string(x.idx) + " overlaps that of tensor " +
                                      std::to_string(other) + (t->projection ? " (or its anchor)" : ""));
    }
    if (x.hi > end_any) {
      end_any = x.hi;
      who_any = x.idx;
    }
    if (x.write && x.hi > end_write) {
      end_write = x.hi;
      who_write = x.idx;
    }
  }
  return DZ_OK;
}

hipError_t upload_chunks(const std::vector<DzChunk>& v, DzChunk** d) {
  if (v.empty()) return hipSuccess;
  hipError_t e = hipMalloc(d, v.size() * sizeof(DzChunk));
  if (e == hipSuccess) e = hipMemcpy(*d, v.data(), v.size() * sizeof(DzChunk), hipMemcpyHostToDevice);
  return e;
}

// The device address of `scratch` on device `dev` (current) and the device's
// CU count, looked up once per device. In host code `scratch` names a host
// stand-in, not device memory: the kernels get this address instead.
struct StaticScratch {
  bool ready = false;
  unsigned char* ptr = nullptr;
  int cus = 0;
};
std::mutex g_static_mu;
StaticScratch g_static[kMaxDevices];

int32_t static_scratch(int dev, StaticScratch** out) {
  std::lock_guard<std::mutex> lk(g_static_mu);
  StaticScratch& s = g_static[dev];
  if (!s.ready) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    e = hipDeviceGetAttribute(&s.cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(MultiprocessorCount)");
    s.ptr = (unsigned char*)p;
    s.ready = true;
  }
  *out = &s;
  return DZ_OK;
}

}  // namespace

extern "C" {

// 3.0.0: z's Philox counter words are (stream, q lo, 0, q hi) (2.0.0: (q lo,
// q hi, stream, 0)); 2.0.0: z from Philox4x32-7 (1.0.0 used Philox4x32-10),
// dz_group_sumsq_static
int32_t dz_version(void) { return 30000; }

const char* dz_last_error(void) { return g_last_error.c_str(); }

int32_t dz_init(int32_t device) {
  int dev;
  int32_t rc = current_device(&dev);
  if (rc) return rc;
  if (device != dev) {
    return fail(DZ_ERR_DEVICE, "dz_init(" + std::to_string(device) + ") with device " + std::to_string(dev) +
                                   " current");
  }
  StaticScratch* sc = nullptr;
  rc = static_scratch(dev, &sc);
  if (rc) return rc;
  // The runtime sets up the library's first kernel launch on a device with an
  // allocation of its own (2 MiB measured): one launch of the plan kernel
  // with an empty batch, which returns at once, takes it here.
  dz::StaticPlanBatch empty{};
  hipError_t e = dz::launch_static_plan(empty, (DzChunk*)(sc->ptr + kStaticOffChunks),
                                        (uint32_t*)(sc->ptr + kStaticOffGroupBegin),
                                        (uint32_t*)(sc->ptr + kStaticOffCounters), nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e != hipSuccess) return hip_fail(e, "dz_init warm-up launch");
  return DZ_OK;
}

int32_t dz_normal_table(int32_t dtype, void* out, int64_t n_entries) {
  if (!valid_dtype(dtype)) return fail(DZ_ERR_INVALID, "unknown dtype");
  if (!out) return fail(DZ_ERR_INVALID, "out is NULL");
  if (n_entries != kDzTabEntries) return fail(DZ_ERR_INVALID, "n_entries must be 32768");
  memcpy(out, host_table_ptr(dtype), (size_t)kDzTabEntries * (size_t)elem_size(dtype));
  return DZ_OK;
}

int32_t dz_philox_host(uint64_t seed, uint32_t stream_id, uint64_t q, uint32_t out[4]) {
  if (!out) return fail(DZ_ERR_INVALID, "out is NULL");
  const DzU4 w = dz_philox_group(seed, stream_id, q);
  out[0] = w.x;
  out[1] = w.y;
  out[2] = w.z;
  out[3] = w.w;
  return DZ_OK;
}

int32_t dz_table_create(const uint64_t* ptrs, const uint64_t* anchor_ptrs, const int64_t* numels,
                        const uint64_t* z_offsets, int32_t n, int32_t dtype, int32_t device, dz_table** out) {
  if (!out) return fail(DZ_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (!ptrs || !numels) return fail(DZ_ERR_INVALID, "ptrs/numels is NULL");
  if (n <= 0 || n > (int32_t)kDzMetaGroupMask) return fail(DZ_ERR_INVALID, "tensor count out of range");
  if (!valid_dtype(dtype)) return fail(DZ_ERR_INVALID, "unknown dtype");
  int cur;
  int32_t rc = current_device(&cur);
  if (rc) return rc;
  if (cur != device) {
    return fail(DZ_ERR_DEVICE, "device " + std::to_string(device) + " is not the current device " +
                                   std::to_string(cur));
  }
  DeviceState* ds = nullptr;
  rc = ensure_device(device, &ds);
  if (rc) return rc;

  dz_table* t = new dz_table();
  t->device = device;
  t->dtype = dtype;
  t->projection = anchor_ptrs != nullptr;
  t->n = n;
  t->dev = ds;
  t->chunk_elems = t->projection ? (uint32_t)dz::proj_chunk_elems(dtype)
                                 : (uint32_t)dz::rmw_chunk_elems(dtype, dz::kModePerturb);
  const int es = elem_size(dtype);
  uint64_t z = 0;
  uint64_t total_tiles = 0;
  for (int32_t i = 0; i < n; ++i) {
    const int64_t ne = numels[i];
    if (ne < 0) {
      free_table(t);
      return fail(DZ_ERR_INVALID, "negative numel for tensor " + std::to_string(i));
    }
    const uint64_t p = ptrs[i];
    const uint64_t a = t->projection ? anchor_ptrs[i] : 0;
    if (z_offsets) {
      if (z_offsets[i] % 8 != 0) {
        free_table(t);
        return fail(DZ_ERR_INVALID, "z offset of tensor " + std::to_string(i) + " is not a multiple of 8");
      }
      z = z_offsets[i];
    }
    if (ne > 0) {
      rc = check_range(p, (uint64_t)ne * es, "theta", i);
      if (!rc && t->projection) rc = check_range(a, (uint64_t)ne * es, "anchor", i);
      if (rc) {
        free_table(t);
        return rc;
      }
    }
    t->ptrs.push_back(p);
    t->aux.push_back(a);
    t->numels.push_back(ne);
    t->zoff.push_back(z);
    // the smallest tile size bounds the tile count
    total_tiles += ((uint64_t)ne + 8191u) / 8192u;
    z += ((uint64_t)ne + 7u) & ~(uint64_t)7u;
  }
  if (total_tiles >= 0xffffffffull) {
    free_table(t);
    return fail(DZ_ERR_INVALID, "too many tiles");
  }
  rc = check_no_overlap(t);
  if (rc) {
    free_table(t);
    return rc;
  }
  std::vector<DzChunk> chunks;
  build_chunks(t, t->chunk_elems, &chunks, t->projection ? &t->group_begin : nullptr);
  t->nchunks = (uint32_t)chunks.size();
  if (!t->projection) (void)full_tiles_first(&chunks, t->chunk_elems);
  hipError_t e = upload_chunks(chunks, &t->d_chunks);
  const uint32_t fused = (uint32_t)dz::rmw_chunk_elems(dtype, dz::kModeRestoreUpdatePerturb);
  if (e == hipSuccess && !t->projection && fused != t->chunk_elems) {
    std::vector<DzChunk> fc;
    build_chunks(t, fused, &fc, nullptr);
    (void)full_tiles_first(&fc, fused);
    t->fused_elems = fused;
    t->fused_nchunks = (uint32_t)fc.size();
    e = upload_chunks(fc, &t->d_fused_chunks);
  }
  if (e == hipSuccess && t->projection) {
    // The finalize kernel always runs, so these exist even with no chunks.
    e = hipMalloc(&t->d_group_begin, t->group_begin.size() * sizeof(uint32_t));
    if (e == hipSuccess)
      e = hipMemcpy(t->d_group_begin, t->group_begin.data(), t->group_begin.size() * sizeof(uint32_t),
                    hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(&t->d_partials, (size_t)(t->nchunks ? t->nchunks : 1) * sizeof(double));
  }
  if (e == hipSuccess) {
    // zeroed once here; every RMW and projection launch leaves them at zero again
    e = hipMalloc(&t->d_counters, dz::kCounterWords * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(t->d_counters, 0, dz::kCounterWords * sizeof(uint32_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
  }
  if (e != hipSuccess) {
    free_table(t);
    return hip_fail(e, "table upload");
  }
  *out = t;
  return DZ_OK;
}

int32_t dz_table_destroy(dz_table* t) {
  if (!t) return DZ_OK;
  int cur = -1;
  (void)hipGetDevice(&cur);
  if (cur != t->device) (void)hipSetDevice(t->device);
  // Kernels may still read the chunk list: wait for the device before freeing.
  hipError_t e = hipDeviceSynchronize();
  free_table(t);
  if (cur >= 0 && cur != t->device) (void)hipSetDevice(cur);
  if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize before table destroy");
  return DZ_OK;
}

int32_t dz_table_matches(const dz_table* t, const uint64_t* ptrs, int32_t n) {
  if (!t || !ptrs) return fail(DZ_ERR_INVALID, "NULL argument");
  if (n != t->n) return 0;
  for (int32_t i = 0; i < n; ++i)
    if (ptrs[i] != t->ptrs[i]) return 0;
  return 1;
}

int32_t dz_table_z_offset(const dz_table* t, int32_t idx, uint64_t* out) {
  if (!t || !out) return fail(DZ_ERR_INVALID, "NULL argument");
  if (idx < 0 || idx >= t->n) return fail(DZ_ERR_INVALID, "tensor index out of range");
  *out = t->zoff[idx];
  return DZ_OK;
}

int32_t dz_table_set_prefetch_min_tiles(dz_table* t, uint32_t min_tiles) {
  int32_t rc = check_table(t);
  if (rc) return rc;
  t->prefetch_min_tiles = min_tiles;
  return DZ_OK;
}

int32_t dz_table_time_next(dz_table* t, void* start_event, void* stop_event) {
  int32_t rc = check_table(t);
  if (rc) return rc;
  t->timing.start = (hipEvent_t)start_event;
  t->timing.stop = (hipEvent_t)stop_event;
  return DZ_OK;
}

int32_t dz_perturb(dz_table* t, uint64_t seed, float scale, float eps, const uint64_t* d_seed, void* stream) {
  dz::DzScalars s{seed, 0, scale, eps, 0.0f, 0.0f};
  dz::DzScalarPtrs p{d_seed, nullptr, nullptr, nullptr};
  return rmw(t, dz::kModePerturb, s, p, stream);
}

int32_t dz_update(dz_table* t, uint64_t seed, float grad, float lr, const uint64_t* d_seed, const void* d_grad,
                  const float* d_lr, void* stream) {
  dz::DzScalars s{seed, 0, 0.0f, 0.0f, grad, lr};
  dz::DzScalarPtrs p{d_seed, nullptr, d_grad, d_lr};
  return rmw(t, dz::kModeUpdate, s, p, stream);
}

int32_t dz_restore_update(dz_table* t, uint64_t seed, float eps, float grad, float lr, const uint64_t* d_seed,
                          const void* d_grad, const float* d_lr, void* stream) {
  dz::DzScalars s{seed, 0, 1.0f, eps, grad, lr};
  dz::DzScalarPtrs p{d_seed, nullptr, d_grad, d_lr};
  return rmw(t, dz::kModeRestoreUpdate, s, p, stream);
}

int32_t dz_restore_update_perturb(dz_table* t, uint64_t seed, uint64_t next_seed, float eps, float grad, float lr,
                                  const uint64_t* d_seed, const uint64_t* d_next_seed, const void* d_grad,
                                  const float* d_lr, void* stream) {
  dz::DzScalars s{seed, next_seed, 1.0f, eps, grad, lr};
  dz::DzScalarPtrs p{d_seed, d_next_seed, d_grad, d_lr};
  return rmw(t, dz::kModeRestoreUpdatePerturb, s, p, stream);
}

int32_t dz_normals(uint64_t seed, uint32_t stream_id, uint64_t offset, int64_t n, int32_t dtype, void* d_out,
                   void* stream) {
  if (!valid_dtype(dtype)) return fail(DZ_ERR_INVALID, "unknown dtype");
  // one thread per element, 256 per block: keep the grid below 2^31 blocks
  if (n < 0 || n > ((int64_t)1 << 38)) return fail(DZ_ERR_INVALID, "n out of range");
  if (n == 0) return DZ_OK;
  int dev;
  int32_t rc = current_device(&dev);
  if (rc) return rc;
  rc = check_range((uint64_t)(uintptr_t)d_out, (uint64_t)n * elem_size(dtype), "out", 0);
  if (rc) return rc;
  DeviceState* ds = nullptr;
  rc = ensure_device(dev, &ds);
  if (rc) return rc;
  hipError_t e = dz::launch_normals(dtype, ds->tab[dtype], seed, stream_id, offset, (uint64_t)n, d_out,
                                    (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "normals kernel launch");
  return DZ_OK;
}

int32_t dz_export_z(const dz_table* t, uint64_t seed, int32_t idx, void* d_out, void* stream) {
  int32_t rc = check_table(t);
  if (rc) return rc;
  if (t->projection) return fail(DZ_ERR_INVALID, "export needs a ZO table");
  if (idx < 0 || idx >= t->n) return fail(DZ_ERR_INVALID, "tensor index out of range");
  return dz_normals(seed, DZ_STREAM_PARAM, t->zoff[idx], t->numels[idx], t->dtype, d_out, stream);
}

int32_t dz_philox(uint64_t seed, uint32_t stream_id, uint64_t q0, int64_t n, uint32_t* d_out, void* stream) {
  if (n < 0 || n > ((int64_t)1 << 36)) return fail(DZ_ERR_INVALID, "n out of range");
  if (n == 0) return DZ_OK;
  int32_t rc = check_range((uint64_t)(uintptr_t)d_out, (uint64_t)n * 16, "out", 0);
  if (rc) return rc;
  hipError_t e = dz::launch_philox(seed, stream_id, q0, (uint64_t)n, d_out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "philox kernel launch");
  return DZ_OK;
}

int32_t dz_group_sumsq(dz_table* t, double* d_sumsq, float* d_norm_f32, void* d_norm_T, void* stream) {
  int32_t rc = check_table(t);
  if (rc) return rc;
  dz::LaunchEvents ev = take_timing(t);
  if (!t->projection) return fail(DZ_ERR_INVALID, "group_sumsq needs a projection table");
  rc = check_group_outputs(t, d_sumsq, d_norm_f32, d_norm_T);
  if (rc) return rc;
  hipError_t e = hipSuccess;
  if (t->nchunks > 0) {
    e = dz::launch_proj(t->dtype, dz::kProjSumsq, t->d_chunks, t->nchunks, (uint32_t)t->n, proj_grid(t),
                        nullptr, t->d_partials, t->d_counters, (hipStream_t)stream, {ev.start, nullptr});
    if (e != hipSuccess) return hip_fail(e, "sumsq kernel launch");
    ev.start = nullptr;
  }
  e = dz::launch_finalize(t->dtype, t->d_partials, t->d_group_begin, (uint32_t)t->n, d_sumsq, d_norm_f32,
                          d_norm_T, true, (hipStream_t)stream, ev);
  if (e != hipSuccess) return hip_fail(e, "finalize kernel launch");
  return DZ_OK;
}

int32_t dz_group_sumsq_static(const uint64_t* ptrs, const uint64_t* anchor_ptrs, const int64_t* numels, int32_t n,
                              int32_t dtype, double* d_sumsq, float* d_norm_f32, void* d_norm_T, void* stream) {
  if (!ptrs || !anchor_ptrs || !numels) return fail(DZ_ERR_INVALID, "ptrs/anchor_ptrs/numels is NULL");
  if (n <= 0 || (uint32_t)n > kStaticMaxGroups) {
    return fail(DZ_ERR_INVALID, "group count must be in [1, " + std::to_string(kStaticMaxGroups) + "]");
  }
  if (!valid_dtype(dtype)) return fail(DZ_ERR_INVALID, "unknown dtype");
  int dev;
  int32_t rc = current_device(&dev);
  if (rc) return rc;
  const int es = elem_size(dtype);
  const uint64_t cn = (uint64_t)dz::proj_chunk_elems(dtype);
  uint64_t total = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (numels[i] < 0) return fail(DZ_ERR_INVALID, "negative numel for tensor " + std::to_string(i));
    total += ((uint64_t)numels[i] + cn - 1) / cn;
  }
  if (total > kStaticMaxChunks) {
    return fail(DZ_ERR_INVALID, "the tensors make " + std::to_string(total) + " chunks of " +
                                    std::to_string(cn) + " elements; at most " +
                                    std::to_string(kStaticMaxChunks) + " fit the static scratch");
  }
  for (int32_t i = 0; i < n; ++i) {
    if (numels[i] > 0) {
      rc = check_range(ptrs[i], (uint64_t)numels[i] * es, "theta", i);
      if (!rc) rc = check_range(anchor_ptrs[i], (uint64_t)numels[i] * es, "anchor", i);
      if (rc) return rc;
    }
  }
  const uint64_t out_bytes[3] = {(uint64_t)n * 8, (uint64_t)n * 4, (uint64_t)n * es};
  const void* outs[3] = {d_sumsq, d_norm_f32, d_norm_T};
  const char* out_names[3] = {"sumsq", "norm_f32", "norm_T"};
  for (int k = 0; k < 3; ++k) {
    if (outs[k]) {
      rc = check_range((uint64_t)(uintptr_t)outs[k], out_bytes[k], out_names[k], 0);
      if (rc) return rc;
    }
  }
  StaticScratch* sc = nullptr;
  rc = static_scratch(dev, &sc);
  if (rc) return rc;
  uint32_t* counters = (uint32_t*)(sc->ptr + kStaticOffCounters);
  uint32_t* group_begin = (uint32_t*)(sc->ptr + kStaticOffGroupBegin);
  DzChunk* chunks = (DzChunk*)(sc->ptr + kStaticOffChunks);
  double* partials = (double*)(sc->ptr + kStaticOffPartials);
  const hipStream_t st = (hipStream_t)stream;
  // the chunk plan, kStaticPlanGroups groups per launch (the group list travels as a kernel argument)
  uint32_t next = 0;
  for (int32_t g0 = 0; g0 < n; g0 += dz::kStaticPlanGroups) {
    dz::StaticPlanBatch b{};
    b.ngroups = (uint32_t)std::min<int32_t>(dz::kStaticPlanGroups, n - g0);
    b.group_base = (uint32_t)g0;
    b.total_groups = (uint32_t)n;
    b.total_chunks = (uint32_t)total;
    b.elem_size = es;
    b.chunk_elems = (int32_t)cn;
    b.first = g0 == 0;
    for (uint32_t k = 0; k < b.ngroups; ++k) {
      b.ptr[k] = ptrs[g0 + k];
      b.anchor[k] = anchor_ptrs[g0 + k];
      b.numel[k] = numels[g0 + k];
      b.chunk_begin[k] = next;
      next += (uint32_t)(((uint64_t)numels[g0 + k] + cn - 1) / cn);
    }
    hipError_t e = dz::launch_static_plan(b, chunks, group_begin, counters, st);
    if (e != hipSuccess) return hip_fail(e, "plan kernel launch");
  }
  if (total > 0) {
    const uint32_t grid = std::min<uint32_t>((uint32_t)total, (uint32_t)sc->cus);
    hipError_t e = dz::launch_proj(dtype, dz::kProjSumsq, chunks, (uint32_t)total, (uint32_t)n, grid, nullptr,
                                   partials, counters, st);
    if (e != hipSuccess) return hip_fail(e, "sumsq kernel launch");
  }
  hipError_t e =
      dz::launch_finalize(dtype, partials, group_begin, (uint32_t)n, d_sumsq, d_norm_f32, d_norm_T, true, st);
  if (e != hipSuccess) return hip_fail(e, "finalize kernel launch");
  return DZ_OK;
}

int32_t dz_project(dz_table* t, const void* d_alpha, int32_t mode, double* d_sumsq, float* d_norm_f32,
                   void* d_norm_T, void* stream) {
  int32_t rc = check_table(t);
  if (rc) return rc;
  dz::LaunchEvents ev = take_timing(t);
  if (!t->projection) return fail(DZ_ERR_INVALID, "project needs a projection table");
  if (mode != DZ_PROJ_APPLY && mode != DZ_PROJ_REVERSE && mode != DZ_PROJ_REVERSE_SUMSQ &&
      mode != DZ_PROJ_APPLY_F32ALPHA)
    return fail(DZ_ERR_INVALID, "mode must be APPLY, REVERSE, REVERSE_SUMSQ or APPLY_F32ALPHA");
  const int alpha_size = mode == DZ_PROJ_APPLY_F32ALPHA ? 4 : elem_size(t->dtype);
  rc = check_range((uint64_t)(uintptr_t)d_alpha, (uint64_t)t->n * alpha_size, "alpha", 0);
  if (!rc) rc = check_group_outputs(t, d_sumsq, d_norm_f32, d_norm_T);
  if (rc) return rc;
  const bool finalize = mode == DZ_PROJ_REVERSE_SUMSQ;
  if (t->nchunks > 0) {
    hipError_t e = dz::launch_proj(t->dtype, mode, t->d_chunks, t->nchunks, (uint32_t)t->n, proj_grid(t),
                                   d_alpha, t->d_partials, t->d_counters, (hipStream_t)stream,
                                   {ev.start, finalize ? nullptr : ev.stop});
    if (e != hipSuccess) return hip_fail(e, "projection kernel launch");
    ev = {nullptr, finalize ? ev.stop : nullptr};
  }
  if (!finalize) return record_unlaunched(ev, stream);
  hipError_t e = dz::launch_finalize(t->dtype, t->d_partials, t->d_group_begin, (uint32_t)t->n, d_sumsq, d_norm_f32,
                                     d_norm_T, true, (hipStream_t)stream, ev);
  if (e != hipSuccess) return hip_fail(e, "finalize kernel launch");
  return DZ_OK;
}

int32_t dz_group_dot(dz_table* t, const uint64_t* other_ptrs, double* d_dot, float* d_dot_f32, void* stream) {
  int32_t rc = check_table(t);
  if (rc) return rc;
  dz::LaunchEvents ev = take_timing(t);
  if (!t->projection) return fail(DZ_ERR_INVALID, "group_dot needs a projection table");
  if (!other_ptrs) return fail(DZ_ERR_INVALID, "other_ptrs is NULL");
  for (int32_t i = 0; i < t->n; ++i) {
    if (t->numels[i] > 0) {
      rc = check_range(other_ptrs[i], (uint64_t)t->numels[i] * elem_size(t->dtype), "other", i);
      if (rc) return rc;
    }
  }
  rc = check_group_outputs(t, d_dot, d_dot_f32, nullptr);
  if (rc) return rc;
  hipError_t e = hipSuccess;
  // one launch per batch of kMaxDotGroups groups (a group's chunks are contiguous)
  for (int32_t g0 = 0; g0 < t->n; g0 += dz::kMaxDotGroups) {
    const int32_t g1 = std::min<int32_t>(t->n, g0 + dz::kMaxDotGroups);
    const uint32_t c0 = t->group_begin[g0], c1 = t->group_begin[g1];
    if (c1 == c0) continue;
    dz::DzPtrArray other{};
    for (int32_t i = g0; i < g1; ++i) other.p[i - g0] = other_ptrs[i];
    e = dz::launch_dot(t->dtype, t->d_chunks + c0, c1 - c0, other, (uint32_t)g0, t->d_partials + c0,
                       (hipStream_t)stream, {ev.start, nullptr});
    if (e != hipSuccess) return hip_fail(e, "dot kernel launch");
    ev.start = nullptr;
  }
  e = dz::launch_finalize(t->dtype, t->d_partials, t->d_group_begin, (uint32_t)t->n, d_dot, d_dot_f32, nullptr,
                          false, (hipStream_t)stream, ev);
  if (e != hipSuccess) return hip_fail(e, "finalize kernel launch");
  return DZ_OK;
}


}  // extern "C"

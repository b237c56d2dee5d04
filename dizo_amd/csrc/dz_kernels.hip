// HIP kernels for the zeroth-order (ZO) step and the DiZO projection, gfx950.
//
// All arithmetic reproduces PyTorch's elementwise recipe bit for bit: every
// operation is one IEEE fp32 operation on fp32-widened operands followed by a
// round-to-nearest-even conversion to the parameter dtype T (identity for
// fp32). Products are never contracted into FMAs (the file is compiled with
// -ffp-contract=off and the pragma below), and dz_opq() keeps the backend from
// folding an fp32 multiply and its fp16 conversion into one mixed-precision
// FMA (which would round once instead of twice and flip the sign of zeros).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dz_common.h"
#include "dz_kernels.h"

#pragma clang fp contract(off)

namespace dz {

// Opaque identity: the value must exist as a plain fp32 register here.
__device__ __forceinline__ float dz_opq(float x) {
  asm("" : "+v"(x));
  return x;
}

template <int DT>
struct DT_;

template <>
struct DT_<DZ_F32> {
  using S = uint32_t;
  static constexpr int kBits = 32;
  __device__ static __forceinline__ float to_f(uint32_t b) { return __uint_as_float(b); }
  __device__ static __forceinline__ uint32_t from_f(float f) { return __float_as_uint(f); }
};

template <>
struct DT_<DZ_F16> {
  using S = uint16_t;
  static constexpr int kBits = 16;
  __device__ static __forceinline__ float to_f(uint32_t b) {
    return dz_opq((float)__builtin_bit_cast(_Float16, (uint16_t)b));
  }
  __device__ static __forceinline__ uint32_t from_f(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)dz_opq(f));
  }
};

template <>
struct DT_<DZ_BF16> {
  using S = uint16_t;
  static constexpr int kBits = 16;
  __device__ static __forceinline__ float to_f(uint32_t b) { return __uint_as_float(b << 16); }
  __device__ static __forceinline__ uint32_t from_f(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)dz_opq(f));
  }
};

// R_T(x): round an fp32 result to T and widen back.
template <int DT>
__device__ __forceinline__ float rt(float x) {
  if constexpr (DT == DZ_F32) {
    return x;
  } else {
    return DT_<DT>::to_f(DT_<DT>::from_f(x));
  }
}

// ---------------------------------------------------------------------------
// Per-element operations (theta and z are fp32-widened values of T).
// ---------------------------------------------------------------------------

// trainer.py:1442   param.data + scaling_factor * z * eps
template <int DT>
__device__ __forceinline__ uint32_t op_perturb(float th, float z, float s, float eps) {
  const float a = rt<DT>(s * z);
  const float b = rt<DT>(a * eps);
  return DT_<DT>::from_f(th + b);
}

// trainer.py:1608   param.data - lr * (projected_grad * z)
template <int DT>
__device__ __forceinline__ uint32_t op_update(float th, float z, float g, float lr) {
  const float c = rt<DT>(g * z);
  const float d = rt<DT>(lr * c);
  return DT_<DT>::from_f(th - d);
}

template <int DT, int MODE>
__device__ __forceinline__ uint32_t op_rmw(uint32_t thb, uint32_t zb, const DzScalars& s) {
  const float th = DT_<DT>::to_f(thb);
  const float z = DT_<DT>::to_f(zb);
  if constexpr (MODE == kModePerturb) {
    return op_perturb<DT>(th, z, s.scale, s.eps);
  } else if constexpr (MODE == kModeUpdate) {
    return op_update<DT>(th, z, s.grad, s.lr);
  } else {  // kModeRestoreUpdate
    // trainer.py:1593 (restore, scaling_factor=+1) then trainer.py:1608.
    const float th1 = DT_<DT>::to_f(op_perturb<DT>(th, z, 1.0f, s.eps));
    return op_update<DT>(th1, z, s.grad, s.lr);
  }
}

// z bits of field j of a Philox block, from the LDS quantile table.
template <int DT>
__device__ __forceinline__ uint32_t z_bits(const typename DT_<DT>::S* tab, uint32_t h) {
  const uint32_t mag = (uint32_t)tab[h & 0x7fffu];
  return mag | ((h & 0x8000u) << (DT_<DT>::kBits - 16));
}

__device__ __forceinline__ uint32_t word_of(const DzU4& w, int i) {
  return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
}

template <int DT>
__device__ __forceinline__ float load_scalar_T(const void* p) {
  return DT_<DT>::to_f((uint32_t)(*(const typename DT_<DT>::S*)p));
}

template <int DT>
__device__ __forceinline__ DzScalars resolve_scalars(DzScalars s, const DzScalarPtrs& p) {
  if (p.seed) s.seed = *p.seed;
  if (p.grad) s.grad = load_scalar_T<DT>(p.grad);
  if (p.lr) s.lr = *p.lr;
  return s;
}

// ---------------------------------------------------------------------------
// Multi-tensor read-modify-write kernel (perturb / update / restore+update).
// Persistent workgroups walk the chunk list; each thread owns kUnroll groups
// of 8 consecutive elements per chunk (one Philox call each). The 15-bit
// quantile table lives in LDS.
// ---------------------------------------------------------------------------
template <int DT, int MODE>
__global__ void __launch_bounds__(kRmwThreads) rmw_kernel(const DzChunk* __restrict__ chunks,
                                                          uint32_t nchunks,
                                                          const void* __restrict__ gtab,
                                                          DzScalars sc_in, DzScalarPtrs sp) {
  using S = typename DT_<DT>::S;
  __shared__ __attribute__((aligned(16))) S tab[kDzTabEntries];
  {
    const uint4* src = (const uint4*)gtab;
    uint4* dst = (uint4*)tab;
    constexpr int kVecs = (int)(kDzTabEntries * sizeof(S) / 16);
    for (int i = threadIdx.x; i < kVecs; i += kRmwThreads) dst[i] = src[i];
  }
  const DzScalars sc = resolve_scalars<DT>(sc_in, sp);
  __syncthreads();

  constexpr int kES = (int)sizeof(S);
  for (uint32_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const DzChunk ch = chunks[c];
    const bool aligned = (ch.meta & kDzMetaAligned) != 0u;
    char* base = (char*)ch.ptr;
    if (ch.n == (uint32_t)kRmwChunk && aligned) {
      if constexpr (kES == 2) {
        uint4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const uint32_t g = threadIdx.x + u * kRmwThreads;
          v[u] = *(const uint4*)(base + (size_t)g * 16);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const uint32_t g = threadIdx.x + u * kRmwThreads;
          const DzU4 w = dz_philox_group(sc.seed, kDzStreamParam, ch.zgroup + g);
          uint32_t in[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
          uint32_t out[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t wi = word_of(w, i);
            const uint32_t z0 = z_bits<DT>(tab, wi & 0xffffu);
            const uint32_t z1 = z_bits<DT>(tab, wi >> 16);
            const uint32_t r0 = op_rmw<DT, MODE>(in[i] & 0xffffu, z0, sc);
            const uint32_t r1 = op_rmw<DT, MODE>(in[i] >> 16, z1, sc);
            out[i] = (r0 & 0xffffu) | (r1 << 16);
          }
          *(uint4*)(base + (size_t)g * 16) = make_uint4(out[0], out[1], out[2], out[3]);
        }
      } else {
        uint4 v[kUnroll][2];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const uint32_t g = threadIdx.x + u * kRmwThreads;
          v[u][0] = *(const uint4*)(base + (size_t)g * 32);
          v[u][1] = *(const uint4*)(base + (size_t)g * 32 + 16);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const uint32_t g = threadIdx.x + u * kRmwThreads;
          const DzU4 w = dz_philox_group(sc.seed, kDzStreamParam, ch.zgroup + g);
          uint32_t in[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w,
                            v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
          uint32_t out[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t h = (word_of(w, j >> 1) >> (16 * (j & 1))) & 0xffffu;
            out[j] = op_rmw<DT, MODE>(in[j], z_bits<DT>(tab, h), sc);
          }
          *(uint4*)(base + (size_t)g * 32) = make_uint4(out[0], out[1], out[2], out[3]);
          *(uint4*)(base + (size_t)g * 32 + 16) = make_uint4(out[4], out[5], out[6], out[7]);
        }
      }
    } else {
      // Partial or misaligned chunk: per-group, per-element with bounds checks.
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t g = threadIdx.x + u * kRmwThreads;
        const uint32_t e0 = g * 8u;
        if (e0 >= ch.n) continue;
        const DzU4 w = dz_philox_group(sc.seed, kDzStreamParam, ch.zgroup + g);
        const uint32_t m = min(8u, ch.n - e0);
        for (uint32_t j = 0; j < m; ++j) {
          const uint32_t h = (word_of(w, (int)(j >> 1)) >> (16 * (j & 1))) & 0xffffu;
          S* p = (S*)(base + (size_t)(e0 + j) * kES);
          *p = (S)op_rmw<DT, MODE>((uint32_t)*p, z_bits<DT>(tab, h), sc);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Projection kernels over the projected (k/v) tensors, one group per tensor.
//   SUMSQ          partial[c] = sum over chunk of fp32(R_T(theta - theta0))^2
//   APPLY          theta <- R_T(R_T(R_T(theta - theta0) * alpha) + theta0)   trainer.py:428-436
//   REVERSE        theta <- R_T(R_T(R_T(theta - theta0) / alpha) + theta0)   trainer.py:447-451
//   REVERSE_SUMSQ  REVERSE, then partial[c] of the new theta (next norm, trainer.py:455-457)
// One chunk per workgroup; squares and sums in fp64 (exact squares of the
// fp32-widened differences); fixed reduction order, so results are deterministic.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ void proj_elem(int mode, uint32_t thb, uint32_t t0b, float alpha,
                                          uint32_t* outb, double* acc) {
  const float th = DT_<DT>::to_f(thb);
  const float t0 = DT_<DT>::to_f(t0b);
  const float d = rt<DT>(th - t0);
  if (mode == kProjSumsq) {
    const double dd = (double)d;
    *acc += dd * dd;
    *outb = thb;
    return;
  }
  float v;
  if (mode == kProjApply) {
    v = rt<DT>(d * alpha);
  } else {
    v = rt<DT>(d / alpha);
  }
  const uint32_t nb = DT_<DT>::from_f(v + t0);
  *outb = nb;
  if (mode == kProjReverseSumsq) {
    const double d2 = (double)rt<DT>(DT_<DT>::to_f(nb) - t0);
    *acc += d2 * d2;
  }
}

__device__ __forceinline__ double block_sum_f64(double x, double* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wid] = x;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0) {
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
  }
  return t;
}

template <int DT, int MODE>
__global__ void __launch_bounds__(kProjThreads) proj_kernel(const DzChunk* __restrict__ chunks,
                                                            const void* __restrict__ alpha_T,
                                                            double* __restrict__ partials) {
  using S = typename DT_<DT>::S;
  constexpr int kES = (int)sizeof(S);
  __shared__ double red[kProjThreads / 64];
  const uint32_t c = blockIdx.x;
  const DzChunk ch = chunks[c];
  const uint32_t grp = ch.meta & kDzMetaGroupMask;
  float alpha = 0.0f;
  if constexpr (MODE != kProjSumsq) alpha = DT_<DT>::to_f((uint32_t)((const S*)alpha_T)[grp]);
  char* tp = (char*)ch.ptr;
  const char* ap = (const char*)ch.aux;
  double acc = 0.0;
  const bool aligned = (ch.meta & kDzMetaAligned) != 0u;
  if (ch.n == (uint32_t)kProjChunk && aligned) {
    constexpr int kPer = 16 / kES;  // elements per 16-byte vector
    constexpr int kVecsPerThread = kProjChunk / (kProjThreads * kPer);
    uint4 vt[kVecsPerThread], va[kVecsPerThread];
#pragma unroll
    for (int u = 0; u < kVecsPerThread; ++u) {
      const size_t off = (size_t)(threadIdx.x + u * kProjThreads) * 16;
      vt[u] = *(const uint4*)(tp + off);
      va[u] = *(const uint4*)(ap + off);
    }
#pragma unroll
    for (int u = 0; u < kVecsPerThread; ++u) {
      const uint32_t it[4] = {vt[u].x, vt[u].y, vt[u].z, vt[u].w};
      const uint32_t ia[4] = {va[u].x, va[u].y, va[u].z, va[u].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kES == 2) {
          uint32_t r0, r1;
          proj_elem<DT>(MODE, it[i] & 0xffffu, ia[i] & 0xffffu, alpha, &r0, &acc);
          proj_elem<DT>(MODE, it[i] >> 16, ia[i] >> 16, alpha, &r1, &acc);
          o[i] = (r0 & 0xffffu) | (r1 << 16);
        } else {
          proj_elem<DT>(MODE, it[i], ia[i], alpha, &o[i], &acc);
        }
      }
      if constexpr (MODE != kProjSumsq) {
        const size_t off = (size_t)(threadIdx.x + u * kProjThreads) * 16;
        *(uint4*)(tp + off) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  } else {
    for (uint32_t e = threadIdx.x; e < ch.n; e += kProjThreads) {
      S* p = (S*)(tp + (size_t)e * kES);
      const S* q = (const S*)(ap + (size_t)e * kES);
      uint32_t r;
      proj_elem<DT>(MODE, (uint32_t)*p, (uint32_t)*q, alpha, &r, &acc);
      if constexpr (MODE != kProjSumsq) *p = (S)r;
    }
  }
  if constexpr (MODE == kProjSumsq || MODE == kProjReverseSumsq) {
    const double t = block_sum_f64(acc, red);
    if (threadIdx.x == 0) partials[c] = t;
  }
}

// Per-group reduction of chunk partials, in chunk order, then
// norm = R_T(sqrt_f32(fp32(sum)))  (torch.norm: fp32 accumulate, fp32 sqrt, cast to T).
template <int DT>
__global__ void __launch_bounds__(kProjThreads) finalize_kernel(const double* __restrict__ partials,
                                                                const uint32_t* __restrict__ gbegin,
                                                                double* __restrict__ sumsq,
                                                                float* __restrict__ norm_f32,
                                                                void* __restrict__ norm_T) {
  using S = typename DT_<DT>::S;
  __shared__ double red[kProjThreads / 64];
  const uint32_t g = blockIdx.x;
  const uint32_t b = gbegin[g], e = gbegin[g + 1];
  double x = 0.0;
  for (uint32_t i = b + threadIdx.x; i < e; i += kProjThreads) x += partials[i];
  const double t = block_sum_f64(x, red);
  if (threadIdx.x == 0) {
    const float n = sqrtf((float)t);
    if (sumsq) sumsq[g] = t;
    if (norm_f32) norm_f32[g] = n;
    if (norm_T) ((S*)norm_T)[g] = (S)DT_<DT>::from_f(n);
  }
}

// z(seed, stream, offset + i) for i < n, written densely in T.
template <int DT>
__global__ void __launch_bounds__(256) normals_kernel(const void* __restrict__ gtab, uint64_t seed,
                                                      uint32_t stream, uint64_t offset, uint64_t n,
                                                      void* __restrict__ out) {
  using S = typename DT_<DT>::S;
  const S* tab = (const S*)gtab;
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t e = offset + i;
  const DzU4 w = dz_philox_group(seed, stream, e >> 3);
  const uint32_t j = (uint32_t)(e & 7u);
  const uint32_t h = (word_of(w, (int)(j >> 1)) >> (16 * (j & 1))) & 0xffffu;
  ((S*)out)[i] = (S)z_bits<DT>(tab, h);
}

// Raw Philox blocks for counter q = q0 + i (test and KAT use).
__global__ void __launch_bounds__(256) philox_kernel(uint64_t seed, uint32_t stream, uint64_t q0,
                                                     uint64_t n, uint32_t* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const DzU4 w = dz_philox_group(seed, stream, q0 + i);
  out[4 * i + 0] = w.x;
  out[4 * i + 1] = w.y;
  out[4 * i + 2] = w.z;
  out[4 * i + 3] = w.w;
}

// ---------------------------------------------------------------------------
// Launchers (host side, C++ linkage; the C ABI validates before calling).
// ---------------------------------------------------------------------------
template <int DT>
static hipError_t launch_rmw_dt(int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t grid,
                                const void* tab, const DzScalars& s, const DzScalarPtrs& p,
                                hipStream_t st) {
  switch (mode) {
    case kModePerturb:
      hipLaunchKernelGGL((rmw_kernel<DT, kModePerturb>), dim3(grid), dim3(kRmwThreads), 0, st,
                         chunks, nchunks, tab, s, p);
      break;
    case kModeUpdate:
      hipLaunchKernelGGL((rmw_kernel<DT, kModeUpdate>), dim3(grid), dim3(kRmwThreads), 0, st,
                         chunks, nchunks, tab, s, p);
      break;
    case kModeRestoreUpdate:
      hipLaunchKernelGGL((rmw_kernel<DT, kModeRestoreUpdate>), dim3(grid), dim3(kRmwThreads), 0,
                         st, chunks, nchunks, tab, s, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rmw(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t grid,
                      const void* tab, const DzScalars& s, const DzScalarPtrs& p, hipStream_t st) {
  switch (dtype) {
    case DZ_F32: return launch_rmw_dt<DZ_F32>(mode, chunks, nchunks, grid, tab, s, p, st);
    case DZ_F16: return launch_rmw_dt<DZ_F16>(mode, chunks, nchunks, grid, tab, s, p, st);
    case DZ_BF16: return launch_rmw_dt<DZ_BF16>(mode, chunks, nchunks, grid, tab, s, p, st);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
static hipError_t launch_proj_dt(int mode, const DzChunk* chunks, uint32_t nchunks, const void* alpha,
                                 double* partials, hipStream_t st) {
  switch (mode) {
    case kProjSumsq:
      hipLaunchKernelGGL((proj_kernel<DT, kProjSumsq>), dim3(nchunks), dim3(kProjThreads), 0, st,
                         chunks, alpha, partials);
      break;
    case kProjApply:
      hipLaunchKernelGGL((proj_kernel<DT, kProjApply>), dim3(nchunks), dim3(kProjThreads), 0, st,
                         chunks, alpha, partials);
      break;
    case kProjReverse:
      hipLaunchKernelGGL((proj_kernel<DT, kProjReverse>), dim3(nchunks), dim3(kProjThreads), 0,
                         st, chunks, alpha, partials);
      break;
    case kProjReverseSumsq:
      hipLaunchKernelGGL((proj_kernel<DT, kProjReverseSumsq>), dim3(nchunks), dim3(kProjThreads),
                         0, st, chunks, alpha, partials);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_proj(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, const void* alpha,
                       double* partials, hipStream_t st) {
  switch (dtype) {
    case DZ_F32: return launch_proj_dt<DZ_F32>(mode, chunks, nchunks, alpha, partials, st);
    case DZ_F16: return launch_proj_dt<DZ_F16>(mode, chunks, nchunks, alpha, partials, st);
    case DZ_BF16: return launch_proj_dt<DZ_BF16>(mode, chunks, nchunks, alpha, partials, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_finalize(int dtype, const double* partials, const uint32_t* gbegin, uint32_t ngroups,
                           double* sumsq, float* norm_f32, void* norm_T, hipStream_t st) {
  switch (dtype) {
    case DZ_F32:
      hipLaunchKernelGGL((finalize_kernel<DZ_F32>), dim3(ngroups), dim3(kProjThreads), 0, st,
                         partials, gbegin, sumsq, norm_f32, norm_T);
      break;
    case DZ_F16:
      hipLaunchKernelGGL((finalize_kernel<DZ_F16>), dim3(ngroups), dim3(kProjThreads), 0, st,
                         partials, gbegin, sumsq, norm_f32, norm_T);
      break;
    case DZ_BF16:
      hipLaunchKernelGGL((finalize_kernel<DZ_BF16>), dim3(ngroups), dim3(kProjThreads), 0, st,
                         partials, gbegin, sumsq, norm_f32, norm_T);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_normals(int dtype, const void* tab, uint64_t seed, uint32_t stream, uint64_t offset,
                          uint64_t n, void* out, hipStream_t st) {
  const uint64_t blocks = (n + 255) / 256;
  switch (dtype) {
    case DZ_F32:
      hipLaunchKernelGGL((normals_kernel<DZ_F32>), dim3((uint32_t)blocks), dim3(256), 0, st, tab,
                         seed, stream, offset, n, out);
      break;
    case DZ_F16:
      hipLaunchKernelGGL((normals_kernel<DZ_F16>), dim3((uint32_t)blocks), dim3(256), 0, st, tab,
                         seed, stream, offset, n, out);
      break;
    case DZ_BF16:
      hipLaunchKernelGGL((normals_kernel<DZ_BF16>), dim3((uint32_t)blocks), dim3(256), 0, st, tab,
                         seed, stream, offset, n, out);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_philox(uint64_t seed, uint32_t stream, uint64_t q0, uint64_t n, uint32_t* out,
                         hipStream_t st) {
  const uint64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(philox_kernel, dim3((uint32_t)blocks), dim3(256), 0, st, seed, stream, q0, n, out);
  return hipGetLastError();
}

}  // namespace dz

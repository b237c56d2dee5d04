// Causal self-attention of an unpadded batch (the ZO step's forwards, which
// run without autograd), for 16-bit T and head dims 64 / 128.
//
// Replaces, for that case, the SDPA call of HF's OPTAttention.forward
// (transformers modeling_opt; reached from the reference's model call in
// forward_wrap_with_option_len, trainer.py:1464). The inputs are the
// projections as the fused k/v/q GEMM leaves them: q unscaled (the kernel
// applies HF's `q * scaling` as R_T(fp32(q) * scaling)), k and v strided
// views of the same buffer. Output: (sequences, L, heads, head_dim), the
// layout HF's attention returns before its reshape.
//
// One 256-thread workgroup per (sequence, head). V is staged transposed in
// LDS, and for L <= 128 K as well (row-major, rows padded by 8 elements), so
// the key loop reads only LDS; for longer sequences both would not leave room
// for two workgroups per CU, and K is read from global memory. Each wave
// takes 32-query blocks and walks the key tiles at or below the diagonal:
//   S^T (32 keys x 32 queries) = K_tile . Q^T      v_mfma_f32_32x32x16_{f16,bf16}
//   O^T (32 dims x 32 queries) += V^T_tile . P^T
// with the softmax in two passes (all scores of a block in registers, then P)
// for L <= 128 and online (running max, rescaled O) for longer sequences.
// Computing the transposed products puts one query in each lane (and its
// lane ^ 32 partner), so the max, the sum and any rescale of O are
// per-lane values, and the S^T accumulator's slots 8c..8c+7 are already the
// B operand of the P^T product over keys 16c..16c+15 of the tile (the V^T
// operand is read with the same key order). P is rounded to T before the
// second product, as flash attention does; softmax and accumulation are fp32.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "dz_common.h"
#include "dz_kernels.h"

namespace dz {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) u32x4_t g_u32x4_t;

constexpr float kLog2e = 1.4426950408889634f;  // 1 / ln 2

template <int DT>
struct AttnT;
template <>
struct AttnT<DZ_F16> {
  __device__ static __forceinline__ float to_f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  __device__ static __forceinline__ uint32_t from_f(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static __forceinline__ f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
  }
};
template <>
struct AttnT<DZ_BF16> {
  __device__ static __forceinline__ float to_f(uint32_t h) { return __uint_as_float(h << 16); }
  __device__ static __forceinline__ uint32_t from_f(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
  }
  __device__ static __forceinline__ f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8_t, a), __builtin_bit_cast(bf8_t, b), c, 0,
                                                   0, 0);
  }
};

__device__ __forceinline__ u32x4_t ld16(const uint16_t* p) { return *(const g_u32x4_t*)(uintptr_t)p; }

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return AttnT<DT>::from_f(lo) | (AttnT<DT>::from_f(hi) << 16);
}

// K goes to LDS up to this length (both tables then fit twice in a CU's LDS).
constexpr int kKLdsMaxLen = 128;

// Row stride of K staged in LDS: 8 elements of padding put the 16-byte
// operand reads of 16 consecutive rows on distinct banks.
template <int HD>
constexpr int kKRow = HD + 8;

__device__ __forceinline__ float max16(const f32x16_t& v) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = fmaxf(v[i], v[i + 8]);
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = fmaxf(a[i], a[i + 4]);
  return fmaxf(fmaxf(a[0], a[2]), fmaxf(a[1], a[3]));
}

__device__ __forceinline__ float sum16(const f32x16_t& v) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = v[i] + v[i + 8];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = a[i] + a[i + 4];
  return (a[0] + a[2]) + (a[1] + a[3]);
}

// S^T tile (32 keys k0.. x 32 queries): lane's A row is key k0 + n, read
// from LDS (ks) or global memory (krow_g); two independent accumulation
// chains (even and odd k-steps) halve the dependent MFMA latency. Keys above
// the query are masked on the diagonal tile. Slot i of the result is key
// k0 + 8 (i / 4) + 4 hf + i % 4.
template <int DT, int HD, bool KL>
__device__ __forceinline__ f32x16_t score_tile(const u32x4_t* bq, const uint16_t* ks, const uint16_t* kbase,
                                               int64_t k_tok, int k0, int n, int hf, bool diag) {
  constexpr int KK = HD / 16;
  u32x4_t ak[KK];
  if constexpr (KL) {
    const uint16_t* krow = ks + (k0 + n) * kKRow<HD> + 8 * hf;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) ak[kk] = *(const u32x4_t*)(krow + 16 * kk);
  } else {
    const uint16_t* krow = kbase + (int64_t)(k0 + n) * k_tok;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) ak[kk] = ld16(krow + 16 * kk);
  }
  f32x16_t s0 = f32x16_t{}, s1 = f32x16_t{};
#pragma unroll
  for (int kk = 0; kk < KK; kk += 2) {
    s0 = AttnT<DT>::mfma(ak[kk], bq[kk], s0);
    if (kk + 1 < KK) s1 = AttnT<DT>::mfma(ak[kk + 1], bq[kk + 1], s1);
  }
  f32x16_t st = s0 + s1;
  if (diag) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (8 * (i >> 2) + 4 * hf + (i & 3) > n) st[i] = -__builtin_inff();
    }
  }
  return st;
}

// O^T += V^T P^T over the 32 keys k0.. of a tile: p holds this lane's 16 P
// values (query n, keys k0 + 8 (i / 4) + 4 hf + i % 4), rounded to T here;
// slots 8c..8c+7 are the B operand over keys k0 + 16c .. +15, and the V^T
// operand (A row = dim 32 t + n) is read in the same key order.
template <int DT, int HD>
__device__ __forceinline__ void pv_tile(f32x16_t* acc, const f32x16_t& p, const uint16_t* vt, int ldr, int k0,
                                        int n, int hf) {
  constexpr int DTL = HD / 32;
  u32x4_t bp[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bp[c][j] = pack2<DT>(p[8 * c + 2 * j], p[8 * c + 2 * j + 1]);
  }
#pragma unroll
  for (int t = 0; t < DTL; ++t) {
    // slots 0..3 / 4..7 = keys k0 + 16 c + 4 hf + 0..3 / + 8 + 0..3
    const uint16_t* vr = vt + (32 * t + n) * ldr + k0 + 4 * hf;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const u32x2_t lo = *(const u32x2_t*)(vr + 16 * c);
      const u32x2_t hi = *(const u32x2_t*)(vr + 16 * c + 8);
      const u32x4_t av = {lo[0], lo[1], hi[0], hi[1]};
      acc[t] = AttnT<DT>::mfma(av, bp[c], acc[t]);
    }
  }
}

// One 32-query block of one (sequence, head); ks is K in LDS when KL.
template <int DT, int HD, bool KL>
__device__ __forceinline__ void attn_block(const AttnArgs& a, const uint16_t* vt, const uint16_t* ks, int ldr,
                                           int64_t seq, int head, int qb) {
  constexpr int KK = HD / 16;  // MFMA k-steps over the head dim
  constexpr int DTL = HD / 32;  // 32-dim tiles of O^T
  const int lane = threadIdx.x & 63;
  const int n = lane & 31, hf = lane >> 5;
  const int q0 = 32 * qb;

  // Q^T as B operands: lane holds query q0 + n, dims 16 kk + 8 hf + 0..7, scaled as HF scales q.
  u32x4_t bq[KK];
  {
    const uint16_t* qrow = a.q + seq * a.q_seq + (int64_t)(q0 + n) * a.q_tok + head * HD + 8 * hf;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u32x4_t x = ld16(qrow + 16 * kk);
      u32x4_t y;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // dz_opq: the fp32 product is rounded to T on its own, as HF's `q * scaling` is
        y[j] = pack2<DT>(dz_opq(AttnT<DT>::to_f(x[j] & 0xffffu) * a.scale),
                         dz_opq(AttnT<DT>::to_f(x[j] >> 16) * a.scale));
      }
      bq[kk] = y;
    }
  }

  f32x16_t acc[DTL];
#pragma unroll
  for (int t = 0; t < DTL; ++t) acc[t] = f32x16_t{};
  const uint16_t* kbase = a.k + seq * a.k_seq + head * HD + 8 * hf;
  float lsum;
  if constexpr (KL) {
    // At most kKLdsMaxLen / 32 key tiles: a block's scores all fit in
    // registers, so the softmax takes two passes (the scores and their max,
    // then P and the products with V) and never rescales the accumulators,
    // which live in AGPRs.
    constexpr int kMaxT = kKLdsMaxLen / 32;
    f32x16_t sc[kMaxT];
    float m = -__builtin_inff();
#pragma unroll
    for (int kt = 0; kt < kMaxT; ++kt) {
      if (kt <= qb) {
        sc[kt] = score_tile<DT, HD, KL>(bq, ks, kbase, a.k_tok, 32 * kt, n, hf, kt == qb);
        m = fmaxf(m, max16(sc[kt]));
      }
    }
    m = fmaxf(m, __shfl_xor(m, 32));
    const float mb = m * kLog2e;
    float ps = 0.0f;
#pragma unroll
    for (int kt = 0; kt < kMaxT; ++kt) {
      if (kt <= qb) {
        f32x16_t p;
#pragma unroll
        for (int i = 0; i < 16; ++i) p[i] = __builtin_amdgcn_exp2f(sc[kt][i] * kLog2e - mb);
        ps += sum16(p);
        pv_tile<DT, HD>(acc, p, vt, ldr, 32 * kt, n, hf);
      }
    }
    lsum = ps + __shfl_xor(ps, 32);
  } else {
    // Longer sequences: online softmax, one key tile at a time.
    float m = -__builtin_inff();
    lsum = 0.0f;
    for (int kt = 0; kt <= qb; ++kt) {
      const f32x16_t st = score_tile<DT, HD, KL>(bq, ks, kbase, a.k_tok, 32 * kt, n, hf, kt == qb);
      float mx = max16(st);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(m, mx);
      const float corr = __builtin_amdgcn_exp2f((m - mnew) * kLog2e);
      const float mb = mnew * kLog2e;
      f32x16_t p;
#pragma unroll
      for (int i = 0; i < 16; ++i) p[i] = __builtin_amdgcn_exp2f(st[i] * kLog2e - mb);
      float ps = sum16(p);
      ps += __shfl_xor(ps, 32);
      lsum = lsum * corr + ps;
      m = mnew;
#pragma unroll
      for (int t = 0; t < DTL; ++t) acc[t] *= corr;
      pv_tile<DT, HD>(acc, p, vt, ldr, 32 * kt, n, hf);
    }
  }

  // O[query q0 + n][dim 32 t + 8 g + 4 hf + 0..3] = acc[t][4 g + 0..3] / lsum
  const float inv = 1.0f / lsum;
  uint16_t* orow = a.out + ((seq * a.L + q0 + n) * (int64_t)a.H + head) * HD + 4 * hf;
#pragma unroll
  for (int t = 0; t < DTL; ++t) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2_t w;
      w[0] = pack2<DT>(dz_opq(acc[t][4 * g] * inv), dz_opq(acc[t][4 * g + 1] * inv));
      w[1] = pack2<DT>(dz_opq(acc[t][4 * g + 2] * inv), dz_opq(acc[t][4 * g + 3] * inv));
      *(u32x2_t*)(orow + 32 * t + 8 * g) = w;
    }
  }
}

// Two waves per SIMD (two workgroups per CU, as the LDS allows).
template <int DT, int HD, bool KL>
__global__ __launch_bounds__(256, 2) void attn_causal_kernel(AttnArgs a) {
  // HD rows of L + 4 keys: V transposed; then, when KL, L rows of K
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* vt = smem;
  const int L = a.L;
  const int ldr = L + 4;
  uint16_t* ks = smem + HD * ldr;
  const int64_t seq = blockIdx.x / a.H;
  const int head = blockIdx.x % a.H;

  // Stage V^T: each thread moves 8 dims of two consecutive keys and writes
  // each dim's pair of keys as one 32-bit word; consecutive lanes take
  // consecutive key pairs, so a wave's writes to one row are contiguous.
  const uint16_t* vbase = a.v + seq * a.v_seq + head * HD;
  uint32_t* vt32 = (uint32_t*)vt;
  for (int idx = threadIdx.x; idx < (L / 2) * (HD / 8); idx += 256) {
    const int kp = idx % (L / 2), c = idx / (L / 2);
    const u32x4_t x0 = ld16(vbase + (int64_t)(2 * kp) * a.v_tok + 8 * c);
    const u32x4_t x1 = ld16(vbase + (int64_t)(2 * kp + 1) * a.v_tok + 8 * c);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      vt32[((8 * c + 2 * j) * ldr) / 2 + kp] = (x0[j] & 0xffffu) | (x1[j] << 16);
      vt32[((8 * c + 2 * j + 1) * ldr) / 2 + kp] = (x0[j] >> 16) | (x1[j] & 0xffff0000u);
    }
  }
  if constexpr (KL) {
    // K row-major, 16-byte chunks; consecutive lanes take consecutive chunks of a row
    const uint16_t* kb = a.k + seq * a.k_seq + head * HD;
    for (int idx = threadIdx.x; idx < L * (HD / 8); idx += 256) {
      const int key = idx / (HD / 8), c = idx % (HD / 8);
      *(u32x4_t*)(ks + key * kKRow<HD> + 8 * c) = ld16(kb + (int64_t)key * a.k_tok + 8 * c);
    }
  }
  __syncthreads();

  // Query blocks of this wave: with <= 4 blocks one each, rotated across
  // workgroups (block b has b + 1 key tiles, so a fixed assignment would load
  // one SIMD with the longest); with more, pairs (p, nqb - 1 - p) of equal total work.
  const int wave = threadIdx.x >> 6;
  const int nqb = L / 32;
  if (nqb <= 4) {
    if (wave < nqb) attn_block<DT, HD, KL>(a, vt, ks, ldr, seq, head, (int)((wave + blockIdx.x) % nqb));
  } else {
    for (int p = wave; p < (nqb + 1) / 2; p += 4) {
      attn_block<DT, HD, KL>(a, vt, ks, ldr, seq, head, p);
      if (nqb - 1 - p != p) attn_block<DT, HD, KL>(a, vt, ks, ldr, seq, head, nqb - 1 - p);
    }
  }
}

}  // namespace

size_t attn_lds_bytes(int head_dim, int L) {
  const size_t v = (size_t)head_dim * (size_t)(L + 4) * 2;
  return L <= kKLdsMaxLen ? v + (size_t)L * (size_t)(head_dim + 8) * 2 : v;
}

// Dynamic LDS above 64 KB has to be allowed per kernel and device; done once
// per (instantiation, device), for the largest size the instantiation takes.
template <int DT, int HD, bool KL>
hipError_t allow_lds() {
  static std::mutex mu;
  static uint64_t done = 0;  // bit d: set on device d
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if ((done >> dev) & 1u) return hipSuccess;
  e = hipFuncSetAttribute((const void*)attn_causal_kernel<DT, HD, KL>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)attn_lds_bytes(HD, KL ? kKLdsMaxLen : 256));
  if (e == hipSuccess) done |= 1ull << dev;
  return e;
}

hipError_t launch_attn_causal(int dtype, int head_dim, const AttnArgs& a, uint32_t nblocks, hipStream_t st) {
  const size_t lds = attn_lds_bytes(head_dim, a.L);
#define DZ_ATTN_CASE(DTV, HDV)                                                                        \
  if (dtype == DTV && head_dim == HDV) {                                                              \
    if (a.L <= kKLdsMaxLen) {                                                                         \
      const hipError_t e = allow_lds<DTV, HDV, true>();                                               \
      if (e != hipSuccess) return e;                                                                  \
      hipLaunchKernelGGL((attn_causal_kernel<DTV, HDV, true>), dim3(nblocks), dim3(256), lds, st, a); \
    } else {                                                                                          \
      const hipError_t e = allow_lds<DTV, HDV, false>();                                              \
      if (e != hipSuccess) return e;                                                                  \
      hipLaunchKernelGGL((attn_causal_kernel<DTV, HDV, false>), dim3(nblocks), dim3(256), lds, st, a);\
    }                                                                                                 \
    return hipGetLastError();                                                                         \
  }
  DZ_ATTN_CASE(DZ_F16, 64)
  DZ_ATTN_CASE(DZ_F16, 128)
  DZ_ATTN_CASE(DZ_BF16, 64)
  DZ_ATTN_CASE(DZ_BF16, 128)
#undef DZ_ATTN_CASE
  return hipErrorInvalidValue;
}

}  // namespace dz

// HIP kernels for the zeroth-order (ZO) step and the DiZO projection, gfx950.
//
// All arithmetic reproduces PyTorch's elementwise recipe bit for bit: every
// operation is one IEEE fp32 operation on fp32-widened operands followed by a
// round-to-nearest-even conversion to the parameter dtype T (identity for
// fp32). Products are never contracted into FMAs (the file is compiled with
// -ffp-contract=off and the pragma below), and dz_opq() keeps the backend from
// folding an fp32 multiply and its fp16 conversion into one mixed-precision
// FMA (which would round once instead of twice and flip the sign of zeros).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "dz_common.h"
#include "dz_kernels.h"

#pragma clang fp contract(off)

namespace dz {

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

template <int DT>
__device__ __forceinline__ float load_scalar_T(const void* p) {
  return DT_<DT>::to_f((uint32_t)(*(const typename DT_<DT>::S*)p));
}

template <int DT>
__device__ __forceinline__ DzScalars resolve_scalars(DzScalars s, const DzScalarPtrs& p) {
  if (p.seed) s.seed = *p.seed;
  if (p.seed2) s.seed2 = *p.seed2;
  if (p.grad) s.grad = load_scalar_T<DT>(p.grad);
  if (p.lr) s.lr = *p.lr;
  return s;
}

__device__ __forceinline__ uint32_t word_of(const DzU4& w, int i) {
  return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
}

// z bits of a 16-bit field h (sign bit + 15-bit index) from a quantile table.
template <int DT>
__device__ __forceinline__ uint32_t z_bits(const typename DT_<DT>::S* tab, uint32_t h) {
  const uint32_t mag = (uint32_t)tab[h & 0x7fffu];
  return mag | ((h & 0x8000u) << (DT_<DT>::kBits - 16));
}

// ---------------------------------------------------------------------------
// Per-launch delta tables.
//
// Every z is +-Q_T[i] for a 15-bit index i, and each of the reference's
// per-element expressions adds an odd function of z to theta:
//   perturb  theta' = R(theta + b),     b = R(R(s*z)*eps)      trainer.py:1442
//   update   theta' = R(theta - d),     d = R(lr*R(g*z))       trainer.py:1608
//                   = R(theta + (-d))   (x - y is x + (-y) in IEEE arithmetic,
//                                        signed zeros included)
// RNE rounding is symmetric in sign, so b(-z) = -b(z) and d(-z) = -d(z). A
// launch evaluates b, or -d, once per table index (32768 entries in LDS, with
// exactly the arithmetic above), and each element then costs one lookup, a
// sign flip and the final add. The fused restore+update keeps the pair
// (b, -d) per entry for 16-bit T. For 16-bit T the final add is done in T:
// fp16 adds natively; bf16 adds in fp32 and rounds to bf16 (the reference's
// own recipe). fp32 carries 24 >= 2p+2 significand bits for p = 11, so the
// fp16 sum rounded once equals the fp32 sum rounded to fp16.
// fp32 tables hold the fp32 delta bits, or for restore+update z itself (the
// pair would not fit in LDS) with b and d evaluated per element.
// ---------------------------------------------------------------------------
template <int DT, int MODE>
struct RmwTraits {
  static constexpr bool kWide = (DT == DZ_F32 || rmw_pair_mode(MODE));
  using E = typename std::conditional<kWide, uint32_t, uint16_t>::type;
  static constexpr int kGroups = rmw_groups(DT, MODE);
  static constexpr int kChunk = rmw_chunk_elems(DT, MODE);
  static constexpr bool kPrefetch = rmw_prefetch_mode(DT, MODE);
};
// Waves per SIMD of an RMW launch: one 1024-thread workgroup per CU, 4 waves
// per SIMD (up to 128 VGPRs per lane).
constexpr int kRmwWavesPerEU = 4;

// bf16 pair tables (restore + update, and with the next perturbation) hold
// each entry's 16-bit halves xor-ed with their own index i: a z field
// h = sign << 15 | i then turns entry i into its signed value with one xor
// against h (i ^ i = 0 and the sign lands on bit 15, the value's sign), which
// a word-selecting xor does for one operand of a packed word at a time
// (xor_hi below). It takes the bf16 three-way pass from 171 to 151 VALU
// instructions per 8-element group; for the single-value bf16 tables of
// perturb and update it measured 0.6-1.8 % slower (HBM-bound passes, same
// box, alternating builds), so they keep plain entries. fp16 applies the
// signs as packed FMA factors.
__host__ __device__ constexpr bool rmw_index_xor(int dt, int mode) {
  return dt == DZ_BF16 && rmw_pair_mode(mode);
}
// What of a z field h is xor-ed into its table entry's halves.
template <int DT, int MODE>
__device__ __forceinline__ uint32_t field_xor(uint32_t h) {
  return rmw_index_xor(DT, MODE) ? (h & 0xffffu) : (h & 0x8000u);
}

// Table entry for z = +Q_T[i] (qbits = bits of Q_T[i]).
template <int DT, int MODE>
__device__ __forceinline__ uint32_t table_entry(uint32_t qbits, const DzScalars& sc) {
  constexpr uint32_t kSign = DT == DZ_F32 ? 0x80000000u : 0x8000u;
  const float z = DT_<DT>::to_f(qbits);
  const float b = rt<DT>(rt<DT>(sc.scale * z) * sc.eps);
  const float d = rt<DT>(sc.lr * rt<DT>(sc.grad * z));
  if constexpr (MODE == kModePerturb) {
    return DT_<DT>::from_f(b);
  } else if constexpr (MODE == kModeUpdate) {
    return DT_<DT>::from_f(d) ^ kSign;
  } else if constexpr (DT == DZ_F32) {
    return qbits;  // restore+update(+perturb) in fp32: z itself
  } else {
    return DT_<DT>::from_f(b) | ((DT_<DT>::from_f(d) ^ kSign) << 16);
  }
}

typedef uint32_t dz_u32x4 __attribute__((ext_vector_type(4)));

// The launch's delta table, built by the 1024 threads of a workgroup in two
// steps: each thread loads its 16-byte slices of Q_T (4 fp32 or 8 16-bit
// entries; slice t + v * 1024), all loads in flight at once (load_table), then
// writes the slices' entries to the same indices of the LDS table
// (store_table). A plain loop of one 32-bit load, a wait and one LDS store
// per entry costs 32 memory latencies in a row per launch.
template <int DT>
struct TableSlices {
  static constexpr int kPer = DT == DZ_F32 ? 4 : 8;  // Q_T entries per 16-byte slice
  static constexpr int kSlices = kDzTabEntries / (kRmwThreads * kPer);
  static_assert(kSlices * kRmwThreads * kPer == kDzTabEntries, "table slices");
  dz_u32x4 q[kSlices];
};

template <int DT>
__device__ __forceinline__ void load_table(TableSlices<DT>& t, const void* qtab) {
#pragma unroll
  for (int v = 0; v < TableSlices<DT>::kSlices; ++v)
    t.q[v] = *(const dz_u32x4*)((const char*)qtab + (size_t)(v * kRmwThreads + threadIdx.x) * 16);
}

template <int DT, int MODE>
__device__ __forceinline__ void store_table(typename RmwTraits<DT, MODE>::E* tab, const TableSlices<DT>& t,
                                            const DzScalars& sc) {
  using E = typename RmwTraits<DT, MODE>::E;
  constexpr int kPer = TableSlices<DT>::kPer;
#pragma unroll
  for (int v = 0; v < TableSlices<DT>::kSlices; ++v) {
    uint32_t e[kPer];
    const uint32_t i0 = (uint32_t)(v * kRmwThreads + threadIdx.x) * kPer;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t w = t.q[v][kPer == 4 ? i : i >> 1];
      const uint32_t qb = kPer == 4 ? w : (i & 1 ? w >> 16 : w & 0xffffu);
      e[i] = table_entry<DT, MODE>(qb, sc);
      if constexpr (rmw_index_xor(DT, MODE)) e[i] ^= (i0 + i) * 0x10001u;
    }
    E* dst = tab + i0;
    if constexpr (sizeof(E) == 4) {
#pragma unroll
      for (int h = 0; h < kPer / 4; ++h) {
        const dz_u32x4 o = {e[4 * h], e[4 * h + 1], e[4 * h + 2], e[4 * h + 3]};
        *(dz_u32x4*)(dst + 4 * h) = o;
      }
    } else {
      const dz_u32x4 o = {e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
      *(dz_u32x4*)dst = o;
    }
  }
}

typedef _Float16 dz_half2 __attribute__((ext_vector_type(2)));
typedef __bf16 dz_bf2 __attribute__((ext_vector_type(2)));

// bf16 lanes of a packed word as fp32 (a bf16 value is the high half of its
// fp32 bit pattern), and two fp32 values rounded to bf16 and packed by one
// v_cvt_pk_bf16_f32 (round to nearest even, as torch converts fp32 to bf16).
__device__ __forceinline__ float bf16_lo_f(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi_f(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const dz_bf2 r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}
// R_bf16(a + b) lane by lane for packed bf16 words, the fp32 sums written out.
__device__ __forceinline__ uint32_t add_pair_bf16(uint32_t a, uint32_t b) {
  return pack_bf16(bf16_lo_f(a) + bf16_lo_f(b), bf16_hi_f(a) + bf16_hi_f(b));
}
// R_bf16(x) as an fp32 value: v_cvt_pk_bf16_f32 with a zero low lane leaves
// the rounded bf16 in the high half and zeros below it, which is the fp32
// bit pattern of the rounded value (no unpacking before the next fp32 add).
// Written as the instruction: from pack_bf16(0.0f, x) the compiler converts
// into the low lane and moves the result up with a v_perm_b32.
__device__ __forceinline__ float round_bf16_f(float x) {
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
  return __uint_as_float(r);
}

// R_T(a + b) for a pair of 16-bit values packed in one word: fp16 adds
// natively (v_pk_add_f16); bf16 adds in fp32 and rounds both lanes with one
// v_cvt_pk_bf16_f32 (RNE). Either equals the reference's fp32 add rounded
// to T: fp32 holds at least 2p + 2 bits of a p-bit format. (Written out for
// bf16: the compiler's own bf16 vector add issued about 5 conversions per
// three-add chain of a word instead of 3.)
template <int DT>
__device__ __forceinline__ uint32_t add_pair(uint32_t a, uint32_t b) {
  if constexpr (DT == DZ_F16) {
    const dz_half2 x = __builtin_bit_cast(dz_half2, a);
    const dz_half2 y = __builtin_bit_cast(dz_half2, b);
    return __builtin_bit_cast(uint32_t, x + y);
  } else {
    return add_pair_bf16(a, b);
  }
}

// Low (pack_lo) or high (pack_hi) 16-bit halves of two words, a's in the low
// lane and b's in the high lane: one v_perm_b32.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// (half EH of e) ^ (half WH of w), placed in the high half over a zero low
// half: the fp32 pattern of the bf16 value it holds. Two high halves are one
// v_bitop3_b32 ((e ^ w) & 0xffff0000); the other forms are one word-selecting
// (SDWA) xor: each source reads bits 0..15 or 16..31 zero-extended, and the
// result's bits 0..15 are written to bits 16..31 with zeros below. (Written
// as the instruction: from the shift-and-xor expression the compiler forms it
// for only some of the uses.)
template <int EH, int WH>
__device__ __forceinline__ float xor_hi(uint32_t e, uint32_t w) {
  uint32_t r;
  if constexpr (EH == 1 && WH == 1)
    r = (e ^ w) & 0xffff0000u;
  else if constexpr (EH == 0 && WH == 0)
    asm("v_xor_b32_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_0"
        : "=v"(r) : "v"(e), "v"(w));
  else if constexpr (EH == 0)
    asm("v_xor_b32_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
        : "=v"(r) : "v"(e), "v"(w));
  else
    asm("v_xor_b32_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0"
        : "=v"(r) : "v"(e), "v"(w));
  return __uint_as_float(r);
}

// R_T(a + b) for one 16-bit value.
template <int DT>
__device__ __forceinline__ uint32_t add_one(uint32_t a, uint32_t b) {
  if constexpr (DT == DZ_F16) {
    const _Float16 r = __builtin_bit_cast(_Float16, (uint16_t)a) + __builtin_bit_cast(_Float16, (uint16_t)b);
    return (uint32_t)__builtin_bit_cast(uint16_t, r);
  } else {
    return DT_<DT>::from_f(__uint_as_float(a << 16) + __uint_as_float(b << 16));
  }
}

// The two table entries indexed by the 15-bit fields of a z word (bits 0..14
// and 16..30; bits 15 and 31 are the signs). The byte offsets index *
// sizeof(E) take three instructions per word: the sign bits are cleared once,
// then each half is shifted into place by a word-selecting (SDWA) shift, which
// reads bits 0..15 or 16..31 of its operand zero-extended (checked on the
// part against the plain mask-and-shift form). Both offsets are at most
// 0x7fff * sizeof(E), inside the table.
template <typename E>
__device__ __forceinline__ void lookup2(const E* tab, uint32_t w, uint32_t& e0, uint32_t& e1) {
  const uint32_t m = w & 0x7fff7fffu;
  uint32_t a0, a1;
  if constexpr (sizeof(E) == 4) {
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
        : "=v"(a0)
        : "v"(m));
    asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
        : "=v"(a1)
        : "v"(m));
  } else {
    asm("v_lshlrev_b32_sdwa %0, 1, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
        : "=v"(a0)
        : "v"(m));
    asm("v_lshlrev_b32_sdwa %0, 1, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
        : "=v"(a1)
        : "v"(m));
  }
  e0 = (uint32_t)*(const E*)((const char*)tab + a0);
  e1 = (uint32_t)*(const E*)((const char*)tab + a1);
}

// Table entries of two 16-bit elements whose z fields are the halves of `w`
// (and, for the step-fused mode, whose next-step z fields are the halves of
// w2): the lookups of one packed word.
struct Entries16 {
  uint32_t e0, e1, f0, f1;
};
template <int DT, int MODE>
__device__ __forceinline__ Entries16 lookup_pair16(uint32_t w, uint32_t w2,
                                                   const typename RmwTraits<DT, MODE>::E* tab) {
  Entries16 t;
  lookup2(tab, w, t.e0, t.e1);
  if constexpr (MODE == kModeRestoreUpdatePerturb) {
    lookup2(tab, w2, t.f0, t.f1);
  } else {
    t.f0 = t.f1 = 0u;
  }
  return t;
}

// The two elements' new values from their entries. A field's sign bit (bit
// 15 of its half) negates its table value: for fp16, once the two lanes'
// values are packed, one xor with w & 0x80008000 (or a +-1.0 factor); for
// bf16 the xor_hi that takes each value to its fp32 pattern.
// R(th + sg * v) lane by lane for sg = +-1.0 (fp16): the product is exact, so
// the fused multiply-add rounds th +- v once, as the add of the negated value does.
__device__ __forceinline__ uint32_t fma_sign_pair(uint32_t sg, uint32_t v, uint32_t th) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(dz_half2, sg),
                                                                __builtin_bit_cast(dz_half2, v),
                                                                __builtin_bit_cast(dz_half2, th)));
}

template <int DT, int MODE>
__device__ __forceinline__ uint32_t combine_pair16(uint32_t th, uint32_t w, uint32_t w2, const Entries16& t) {
  if constexpr (DT == DZ_F16 && rmw_pair_mode(MODE)) {
    // entry = b | (-d) << 16 for a positive z; the signs enter as factors
    // +-1.0 of packed fused multiply-adds (fma_sign_pair), one per add.
    // +-1.0 in each lane: (w & 0x80008000) | 0x3c003c00 as one three-input
    // bitwise op (truth table 0xEA: src0 & src1 | src2)
    const uint32_t sg = __builtin_amdgcn_bitop3_b32(w, 0x80008000u, 0x3c003c00u, 0xEA);
    uint32_t r = fma_sign_pair(sg, pack_hi(t.e0, t.e1), fma_sign_pair(sg, pack_lo(t.e0, t.e1), th));
    if constexpr (MODE == kModeRestoreUpdatePerturb) {
      const uint32_t sg2 = __builtin_amdgcn_bitop3_b32(w2, 0x80008000u, 0x3c003c00u, 0xEA);
      r = fma_sign_pair(sg2, pack_lo(t.f0, t.f1), r);
    }
    return r;
  }
  if constexpr (!rmw_pair_mode(MODE)) {
    return add_pair<DT>(th, (t.e0 | (t.e1 << 16)) ^ (w & 0x80008000u));
  } else {
    // bf16 pairs: entry i = (b ^ i) | ((-d) ^ i) << 16 for a positive z. Each
    // signed value comes out as its fp32 pattern from one xor_hi against the
    // element's z half (element 0: bits 0..15 of w, element 1: bits 16..31).
    // The three adds are the reference's fp32 adds, each rounded to bf16
    // (round_bf16_f for the first two, one packing conversion for the last).
    float lo = round_bf16_f(bf16_lo_f(th) + xor_hi<0, 0>(t.e0, w));
    float hi = round_bf16_f(bf16_hi_f(th) + xor_hi<0, 1>(t.e1, w));
    if constexpr (MODE == kModeRestoreUpdatePerturb) {
      lo = round_bf16_f(lo + xor_hi<1, 0>(t.e0, w));
      hi = round_bf16_f(hi + xor_hi<1, 1>(t.e1, w));
      // the next step's +1 perturbation uses the same b (same scale and eps)
      return pack_bf16(lo + xor_hi<0, 0>(t.f0, w2), hi + xor_hi<0, 1>(t.f1, w2));
    } else {
      return pack_bf16(lo + xor_hi<1, 0>(t.e0, w), hi + xor_hi<1, 1>(t.e1, w));
    }
  }
}

// One element with 16-bit z field h (and next-step field h2).
template <int DT, int MODE>
__device__ __forceinline__ uint32_t apply_one(uint32_t th, uint32_t h, uint32_t h2,
                                              const typename RmwTraits<DT, MODE>::E* tab, const DzScalars& sc) {
  if constexpr (DT == DZ_F32) {
    const uint32_t e = tab[h & 0x7fffu] ^ ((h & 0x8000u) << 16);
    if constexpr (!rmw_pair_mode(MODE)) {
      return __float_as_uint(__uint_as_float(th) + __uint_as_float(e));
    } else {
      const float z = __uint_as_float(e);
      const float th1 = __uint_as_float(op_perturb<DZ_F32>(__uint_as_float(th), z, 1.0f, sc.eps));
      const uint32_t r = op_update<DZ_F32>(th1, z, sc.grad, sc.lr);
      if constexpr (MODE == kModeRestoreUpdatePerturb) {
        const float z2 = __uint_as_float(tab[h2 & 0x7fffu] ^ ((h2 & 0x8000u) << 16));
        return op_perturb<DZ_F32>(__uint_as_float(r), z2, 1.0f, sc.eps);
      }
      return r;
    }
  } else if constexpr (!rmw_pair_mode(MODE)) {
    return add_one<DT>(th, (uint32_t)tab[h & 0x7fffu] ^ field_xor<DT, MODE>(h));
  } else {
    const uint32_t e = tab[h & 0x7fffu] ^ (field_xor<DT, MODE>(h) * 0x10001u);
    uint32_t r = add_one<DT>(add_one<DT>(th, e & 0xffffu), e >> 16);
    if constexpr (MODE == kModeRestoreUpdatePerturb) {
      r = add_one<DT>(r, (tab[h2 & 0x7fffu] ^ field_xor<DT, MODE>(h2)) & 0xffffu);
    }
    return r;
  }
}

// Streaming 16-byte accesses: theta is touched once per pass, so loads and
// stores carry the non-temporal hint. The pointers are global-memory ones
// (address space 1): the accesses then compile to global_load / global_store,
// which count only against the vector-memory wait counter. As generic (FLAT)
// accesses they would also count against the LDS counter, and every wait for
// an LDS table lookup would then wait for the tile loads in flight as well.
typedef __attribute__((address_space(1))) dz_u32x4 dz_global_u32x4;
typedef __attribute__((address_space(1))) char dz_global_char;
__device__ __forceinline__ dz_u32x4 ld_stream(const void* p) {
  return __builtin_nontemporal_load((const dz_global_u32x4*)(uintptr_t)p);
}
__device__ __forceinline__ void st_stream(void* p, dz_u32x4 v) {
  __builtin_nontemporal_store(v, (dz_global_u32x4*)(uintptr_t)p);
}

// Wave-uniform copy of a 32-bit value in a scalar register.
// __builtin_amdgcn_readfirstlane returns a signed int: cast back to uint32_t
// before widening, or values >= 2^31 would sign-extend.
__device__ __forceinline__ uint32_t rfl_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}
__device__ __forceinline__ uint64_t rfl_u64(uint64_t x) {
  return ((uint64_t)rfl_u32((uint32_t)(x >> 32)) << 32) | (uint64_t)rfl_u32((uint32_t)x);
}

// Workgroup barrier that orders LDS accesses only. __syncthreads() is a
// barrier between release and acquire fences on every address space, so
// before the barrier each wave waits for all of its vector-memory operations
// (s_waitcnt vmcnt(0)), its global stores included. The projection kernel's
// barriers only hand over LDS state (the chunk and descriptor rings, the
// reduction slots), and its chunks' stores need no ordering with the other
// waves (chunks are disjoint and nothing in the launch reads them back), so
// its barriers wait for the LDS counter alone. (Measured at OPT-13B: the
// reverse + norm pass, whose reduction barrier comes after the chunk's
// stores, 1.98 -> 1.91 ms; the other projection passes unchanged. The RMW
// kernel's tile loop measured no faster with the same change, since a tile's
// loads complete behind the previous tile's stores either way, so it keeps
// __syncthreads().)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Work tickets of the projection kernel's loop: lane 0 takes the next index
// from a work counter with a returning vector atomic add, issued as an
// instruction of its own so that the compiler's wait-counter bookkeeping does
// not track it, and ticket_wait<N> waits for it explicitly once N more
// vector-memory operations have been issued behind it (the chunk's loads and
// stores). Tracked by the compiler, the ticket's result, read where the full
// and partial chunk paths merge, is waited for with a wait for every
// operation in flight (the chunk's stores included). Hidden from the
// compiler, the ticket only ever makes the compiler's own waits wait for one
// operation more than they count, never less: vector-memory operations leave
// the wait counter in issue order.
//
// The register the atomic writes is not ready until that wait, which the
// compiler does not know: nothing between the two statements may read, copy
// or spill it. ticket_wait takes no operands (a wait that took the ticket as
// an operand, one per chunk path, made the compiler copy the register into
// the merged value's register ahead of the wait), and the value is used only
// through ticket_ready, after the waits. tests/test_kernel_asm.py checks the
// library's generated code for any instruction between the atomic and its
// wait that touches the register.
__device__ __forceinline__ uint32_t ticket_take(uint32_t* counter) {
  uint32_t t;
  asm volatile("global_atomic_add %0, %1, %2, off sc0" : "=&v"(t) : "v"(counter), "v"(1u) : "memory");
  return t;
}
// Waits until at most N vector-memory operations are in flight: the ticket,
// issued before at least N operations that follow it, has returned.
template <int N>
__device__ __forceinline__ void ticket_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// The ticket as a value the compiler may use: an empty volatile statement
// that redefines it, placed after the waits. Volatile statements keep their
// order, so no use of the returned value is scheduled above a wait (a use of
// the atomic's own output could be: the waits have no operands).
__device__ __forceinline__ uint32_t ticket_ready(uint32_t t) {
  asm volatile("" : "+v"(t));
  return t;
}

// A chunk descriptor read from LDS is the same for every lane: move it to
// scalar registers so tile addresses are formed once per wave.
__device__ __forceinline__ DzChunk uniform_chunk(const DzChunk& c) {
  DzChunk u;
  u.ptr = rfl_u64(c.ptr);
  u.aux = 0;
  u.zgroup = rfl_u64(c.zgroup);
  u.n = rfl_u32(c.n);
  u.meta = rfl_u32(c.meta);
  return u;
}

// The same for a projection chunk, whose anchor address (aux) is used and
// whose z group is not.
__device__ __forceinline__ DzChunk uniform_proj_chunk(const DzChunk& c) {
  DzChunk u;
  u.ptr = rfl_u64(c.ptr);
  u.aux = rfl_u64(c.aux);
  u.zgroup = 0;
  u.n = rfl_u32(c.n);
  u.meta = rfl_u32(c.meta);
  return u;
}

// Registers of one full tile: kVecs 16-byte vectors per thread.
template <int DT, int MODE>
struct TileRegs {
  static constexpr int kVecs = (DT == DZ_F32 ? 2 : 1) * RmwTraits<DT, MODE>::kGroups;
  dz_u32x4 v[kVecs];
};

template <int DT, int MODE>
__device__ __forceinline__ bool full_tile(const DzChunk& ch) {
  return ch.n == (uint32_t)RmwTraits<DT, MODE>::kChunk && (ch.meta & kDzMetaAligned) != 0u;
}

// Lane layout of a full tile: a thread's groups of 8 elements are
// threadIdx.x + u * 1024 for u < G (tile-local group indices), so each load
// instruction of the workgroup covers contiguous memory. at(i) is the byte
// offset of the thread's vector i from the tile's start: group u = i (16-bit)
// or i / 2 (fp32, two vectors per group). A tile holds at most 64 KB. The
// offsets are loop-invariant 64-bit values, so each access adds one to the
// tile's base (one v_lshl_add_u64).
template <int DT, int MODE>
struct TileOffsets {
  __device__ __forceinline__ size_t at(int i) const {
    const size_t g0 = threadIdx.x;
    return DT != DZ_F32 ? (g0 + (size_t)i * kRmwThreads) * 16 : (g0 + (size_t)(i >> 1) * kRmwThreads) * 32 + (size_t)(i & 1) * 16;
  }
};

template <int DT, int MODE>
__device__ __forceinline__ void load_tile_at(uint64_t addr, const TileOffsets<DT, MODE>& to, TileRegs<DT, MODE>& r) {
#pragma unroll
  for (int i = 0; i < TileRegs<DT, MODE>::kVecs; ++i) r.v[i] = ld_stream((const char*)addr + to.at(i));
}

// Philox block of group threadIdx.x + u * 1024 of a tile: counter zgroup +
// that group. kUniformHi: the counters' high words agree across the tile (the
// low word does not wrap inside it), so the high word is wave-uniform and the
// counter's other uniform words keep round 0 and a product of rounds 1 and 2
// on the scalar unit.
template <bool kUniformHi>
__device__ __forceinline__ DzU4 tile_block(const DzChunk& ch, uint64_t seed, int u) {
  const uint32_t g = threadIdx.x + (uint32_t)u * kRmwThreads;
  if constexpr (kUniformHi) {
    return dz_philox_counter(seed, kDzStreamParam, (uint32_t)ch.zgroup + g, (uint32_t)(ch.zgroup >> 32));
  } else {
    return dz_philox_group(seed, kDzStreamParam, ch.zgroup + g);
  }
}

// Group u of a full fp32 tile with its z words w (and next-step words w2):
// the launch's operation applied and the group stored.
template <int DT, int MODE>
__device__ __forceinline__ void apply_store_group32(uint64_t base, const TileOffsets<DT, MODE>& to,
                                                    const TileRegs<DT, MODE>& r, int u,
                                                    const DzU4& w, const DzU4& w2,
                                                    const typename RmwTraits<DT, MODE>::E* tab, const DzScalars& sc) {
  const dz_u32x4 a = r.v[2 * u], b = r.v[2 * u + 1];
  dz_u32x4 o0, o1;
  o0.x = apply_one<DT, MODE>(a.x, w.x & 0xffffu, w2.x & 0xffffu, tab, sc);
  o0.y = apply_one<DT, MODE>(a.y, w.x >> 16, w2.x >> 16, tab, sc);
  o0.z = apply_one<DT, MODE>(a.z, w.y & 0xffffu, w2.y & 0xffffu, tab, sc);
  o0.w = apply_one<DT, MODE>(a.w, w.y >> 16, w2.y >> 16, tab, sc);
  o1.x = apply_one<DT, MODE>(b.x, w.z & 0xffffu, w2.z & 0xffffu, tab, sc);
  o1.y = apply_one<DT, MODE>(b.y, w.z >> 16, w2.z >> 16, tab, sc);
  o1.z = apply_one<DT, MODE>(b.z, w.w & 0xffffu, w2.w & 0xffffu, tab, sc);
  o1.w = apply_one<DT, MODE>(b.w, w.w >> 16, w2.w >> 16, tab, sc);
  st_stream((char*)base + to.at(2 * u), o0);
  st_stream((char*)base + to.at(2 * u + 1), o1);
}

// A thread's share of a full tile as one straight-line block: the Philox
// blocks of all its groups, then the lookups, adds and stores. Keeping both
// in one basic block (the branch on the counters' high word is taken once
// per tile, outside it) lets the scheduler overlap the ALU work of the Philox
// chains with the LDS lookups; with the chains in a block of their own the
// two ran one after the other (three-way pass at OPT-13B: 8.9 -> 8.2 ms at
// equal Philox rounds).
// kLoadNext (the prefetching tile loop): the next tile's loads, from nptr
// into *nxt, go out once the first group is stored (for one group per
// thread, before the Philox chains), held there by scheduling barriers.
// Measured at OPT-13B fp16, three-way pass, kernel microbench, same box,
// alternating builds: 7.86-7.90 ms with the loads issued before the Philox
// chains, 7.69-7.70 after them, 7.58-7.59 half-way, 7.59 a quarter in, 7.60
// three quarters in, and 7.89 with one vector loaded after each group's
// store; OPT-30B bf16 20.10-20.16 -> 19.83-19.89 ms half-way. In the ZO step
// (the bench's 20-step command, three alternating runs each), where the pass
// follows the GEMMs at a lower clock, after the first of four groups
// 7.63-7.66 ms, half-way 7.73-7.78, three quarters in 7.68-7.72; with three
// groups (bf16) after the first and after the second measured the same.
// Issued at the start, the next tile's reads meet this tile's first stores in
// the memory system (rocprofv3 counts 18 % fewer reads in flight and 2.7
// times the L2 tag stalls per cycle of the perturb pass).
template <int DT, int MODE, bool kUniformHi, bool kLoadNext = false>
__device__ __forceinline__ void tile_body(const DzChunk& ch, const TileOffsets<DT, MODE>& to,
                                          const TileRegs<DT, MODE>& r,
                                          const typename RmwTraits<DT, MODE>::E* tab, const DzScalars& sc,
                                          uint64_t nptr = 0, TileRegs<DT, MODE>* nxt = nullptr) {
  constexpr int G = RmwTraits<DT, MODE>::kGroups;
  // the next tile's loads go out after group kLoadAfter's stores (-1: first)
  constexpr int kLoadAfter = G > 1 ? 0 : -1;
  if constexpr (kLoadNext && kLoadAfter < 0) {
    load_tile_at<DT, MODE>(nptr, to, *nxt);
    __builtin_amdgcn_sched_barrier(0);
  }
  constexpr bool kTwoSeeds = MODE == kModeRestoreUpdatePerturb;
  const uint64_t base = ch.ptr;
  DzU4 w[G], w2[G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    w[u] = tile_block<kUniformHi>(ch, sc.seed, u);
    w2[u] = kTwoSeeds ? tile_block<kUniformHi>(ch, sc.seed2, u) : w[u];
  }
#pragma unroll
  for (int u = 0; u < G; ++u) {
    if constexpr (DT == DZ_F32) {
      apply_store_group32<DT, MODE>(base, to, r, u, w[u], w2[u], tab, sc);
    } else {
      dz_u32x4 o;
      o.x = combine_pair16<DT, MODE>(r.v[u].x, w[u].x, w2[u].x, lookup_pair16<DT, MODE>(w[u].x, w2[u].x, tab));
      o.y = combine_pair16<DT, MODE>(r.v[u].y, w[u].y, w2[u].y, lookup_pair16<DT, MODE>(w[u].y, w2[u].y, tab));
      o.z = combine_pair16<DT, MODE>(r.v[u].z, w[u].z, w2[u].z, lookup_pair16<DT, MODE>(w[u].z, w2[u].z, tab));
      o.w = combine_pair16<DT, MODE>(r.v[u].w, w[u].w, w2[u].w, lookup_pair16<DT, MODE>(w[u].w, w2[u].w, tab));
      st_stream((char*)base + to.at(u), o);
    }
    if constexpr (kLoadNext && kLoadAfter >= 0) {
      if (u == kLoadAfter) {
        __builtin_amdgcn_sched_barrier(0);
        load_tile_at<DT, MODE>(nptr, to, *nxt);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

// Whether the Philox counters of a full tile's groups share their high word
// (the low word does not wrap inside the tile).
template <int DT, int MODE>
__device__ __forceinline__ bool tile_counters_share_high_word(const DzChunk& ch) {
  constexpr uint32_t kSpan = (uint32_t)(RmwTraits<DT, MODE>::kGroups * kRmwThreads);
  return (uint32_t)ch.zgroup <= 0xffffffffu - (kSpan - 1u);
}

// Whether the prefetching tile loop can take a tile: a full tile whose
// Philox counters share their high word.
template <int DT, int MODE>
__device__ __forceinline__ bool prefetchable_tile(const DzChunk& ch) {
  return full_tile<DT, MODE>(ch) && tile_counters_share_high_word<DT, MODE>(ch);
}

// Take bit of the RMW kernel's LDS descriptor ring: the top bit of a slot's
// Philox group (a group index is an element index / 8, so its top three bits
// are always clear), set when the slot holds a valid tile that
// prefetchable_tile accepts. bf16 launches that run the prefetching loop set
// it (ring_tagged); every reader of their ring clears it.
constexpr uint64_t kRingTake = 1ull << 63;

// Whether the prefetching loop's ring carries take bits: bf16 only, whose
// three-way pass is VALU-bound (1.4-1.9 % faster with them); the fp16 pass,
// which is not, measured 0.1 % slower.
__host__ __device__ constexpr bool ring_tagged(int dtype) { return dtype == DZ_BF16; }

// The next tile's descriptor as the prefetching loop's steps read it from the
// ring: the address and the Philox group with its take bit. n and meta are
// not read (0 here): the loop's body does not use them.
__device__ __forceinline__ DzChunk uniform_next_chunk(const DzChunk& c) {
  DzChunk u;
  u.ptr = rfl_u64(c.ptr);
  u.aux = 0;
  u.zgroup = rfl_u64(c.zgroup);
  u.n = 0;
  u.meta = 0;
  return u;
}

// Applies the launch's operation to a thread's share of a full tile, already
// in registers, and stores it.
template <int DT, int MODE>
__device__ __forceinline__ void compute_store_tile(const DzChunk& ch, const TileOffsets<DT, MODE>& to,
                                                   const TileRegs<DT, MODE>& r,
                                                   const typename RmwTraits<DT, MODE>::E* tab,
                                                   const DzScalars& sc) {
  if (tile_counters_share_high_word<DT, MODE>(ch)) {
    tile_body<DT, MODE, true>(ch, to, r, tab, sc);
  } else {
    tile_body<DT, MODE, false>(ch, to, r, tab, sc);
  }
}

// Partial or misaligned tile, bounds-checked: groups threadIdx.x,
// threadIdx.x + 1024, ... of the tile. In a 16-byte-aligned tensor a group
// with all 8 elements inside the tile goes through vector loads and stores
// like a full tile's; the tensor's last, incomplete group and every group of
// a misaligned view go element by element.
template <int DT, int MODE>
__device__ __forceinline__ void rmw_partial(const DzChunk& ch, const typename RmwTraits<DT, MODE>::E* tab,
                                            const DzScalars& sc) {
  using S = typename DT_<DT>::S;
  constexpr bool kTwoSeeds = MODE == kModeRestoreUpdatePerturb;
  char* base = (char*)ch.ptr;
  const bool aligned = (ch.meta & kDzMetaAligned) != 0u;
  for (uint32_t g = threadIdx.x; g * 8u < ch.n; g += kRmwThreads) {
    const DzU4 w = dz_philox_group(sc.seed, kDzStreamParam, ch.zgroup + g);
    const DzU4 w2 = kTwoSeeds ? dz_philox_group(sc.seed2, kDzStreamParam, ch.zgroup + g) : w;
    if (aligned && (g + 1u) * 8u <= ch.n) {
      if constexpr (DT == DZ_F32) {
        char* p = base + (size_t)g * 32;
        const dz_u32x4 a = ld_stream(p), b = ld_stream(p + 16);
        dz_u32x4 o0, o1;
        o0.x = apply_one<DT, MODE>(a.x, w.x & 0xffffu, w2.x & 0xffffu, tab, sc);
        o0.y = apply_one<DT, MODE>(a.y, w.x >> 16, w2.x >> 16, tab, sc);
        o0.z = apply_one<DT, MODE>(a.z, w.y & 0xffffu, w2.y & 0xffffu, tab, sc);
        o0.w = apply_one<DT, MODE>(a.w, w.y >> 16, w2.y >> 16, tab, sc);
        o1.x = apply_one<DT, MODE>(b.x, w.z & 0xffffu, w2.z & 0xffffu, tab, sc);
        o1.y = apply_one<DT, MODE>(b.y, w.z >> 16, w2.z >> 16, tab, sc);
        o1.z = apply_one<DT, MODE>(b.z, w.w & 0xffffu, w2.w & 0xffffu, tab, sc);
        o1.w = apply_one<DT, MODE>(b.w, w.w >> 16, w2.w >> 16, tab, sc);
        st_stream(p, o0);
        st_stream(p + 16, o1);
      } else {
        char* p = base + (size_t)g * 16;
        const dz_u32x4 v = ld_stream(p);
        dz_u32x4 o;
        o.x = combine_pair16<DT, MODE>(v.x, w.x, w2.x, lookup_pair16<DT, MODE>(w.x, w2.x, tab));
        o.y = combine_pair16<DT, MODE>(v.y, w.y, w2.y, lookup_pair16<DT, MODE>(w.y, w2.y, tab));
        o.z = combine_pair16<DT, MODE>(v.z, w.z, w2.z, lookup_pair16<DT, MODE>(w.z, w2.z, tab));
        o.w = combine_pair16<DT, MODE>(v.w, w.w, w2.w, lookup_pair16<DT, MODE>(w.w, w2.w, tab));
        st_stream(p, o);
      }
      continue;
    }
    const uint32_t m = min(8u, ch.n - g * 8u);
    for (uint32_t j = 0; j < m; ++j) {
      const uint32_t h = (word_of(w, (int)(j >> 1)) >> (16 * (j & 1))) & 0xffffu;
      const uint32_t h2 = (word_of(w2, (int)(j >> 1)) >> (16 * (j & 1))) & 0xffffu;
      S* p = (S*)(base + (size_t)(g * 8u + j) * sizeof(S));
      *p = (S)apply_one<DT, MODE>((uint32_t)*p, h, h2, tab, sc);
    }
  }
}

// ---------------------------------------------------------------------------
// Multi-tensor read-modify-write kernel (perturb / update / restore+update).
// Persistent workgroups (one per CU) build the launch's delta table in LDS,
// then take tiles from the table's counters, handed out dynamically: that
// keeps the work in flight close together in memory and lets fast
// workgroups take more, which a static grid-stride split does not. The
// workgroup takes whole tiles from counters j of K = min(8, grid / 8),
// workgroup b using counter (b / 8) mod K, so every counter serves
// workgroups on every XCD; wave 0 keeps a ring in LDS (while tile k streams,
// the index of tile k+3 is taken and the descriptor of tile k+2 is loaded,
// with scalar loads) and a barrier ends each tile. The chunk list holds its
// full, aligned tiles first. The last workgroup to finish resets the
// counters for the next launch.
//
// Two tile loops: the plain loop (rmw_tiles) loads each tile when its turn
// comes; the prefetching loop (rmw_tiles_prefetch, the restore + update +
// next perturb passes; a table can set a minimum launch size,
// dz_table_set_prefetch_min_tiles) issues the next full tile's loads once
// each tile's first group is stored, and hands the workgroup's remaining
// tiles to rmw_tiles at its first tile that is not full.
// ---------------------------------------------------------------------------
template <int DT, int MODE, bool kTagged = false>
__device__ __forceinline__ void rmw_tiles(uint32_t k0, const DzChunk* __restrict__ chunks, uint32_t nchunks,
                                          const typename RmwTraits<DT, MODE>::E* tab, const DzScalars& sc,
                                          const TileOffsets<DT, MODE>& to, uint32_t* sidx, DzChunk* sdesc,
                                          uint32_t* mine, uint32_t ncnt, uint32_t j) {
  const uint64_t nch = nchunks;
  TileRegs<DT, MODE> cur;
  for (uint32_t k = k0;; ++k) {
    const uint32_t c = sidx[k % 4];
    if (c >= nchunks) break;
    DzChunk ch = uniform_chunk(sdesc[k % 3]);
    if constexpr (kTagged) ch.zgroup &= ~kRingTake;
    // Wave 0 fetches a descriptor with scalar loads (it is uniform, so it
    // costs no vector registers); lane 0 takes an index with a vector
    // atomic. The anchor field is unused by ZO tables.
    uint32_t grabbed = 0;
    uint64_t n_ptr = 0, n_zg = 0;
    uint32_t n_n = 0, n_meta = 0;
    bool have_desc = false;
    if ((rfl_u32(threadIdx.x) >> 6) == 0) {  // wave 0 (uniform branch)
      if (threadIdx.x == 0) grabbed = atomicAdd(mine, 1u);
      const uint32_t cd = rfl_u32(sidx[(k + 2) % 4]);
      if (cd < nchunks) {
        const DzChunk* src = chunks + cd;
        n_ptr = src->ptr;
        n_zg = src->zgroup;
        n_n = src->n;
        n_meta = src->meta;
        have_desc = true;
      }
    }
    if (full_tile<DT, MODE>(ch)) {
      load_tile_at<DT, MODE>(ch.ptr, to, cur);
      compute_store_tile<DT, MODE>(ch, to, cur, tab, sc);
    } else {
      rmw_partial<DT, MODE>(ch, tab, sc);
    }
    if (threadIdx.x == 0) {
      sidx[(k + 3) % 4] = (uint32_t)min((uint64_t)grabbed * ncnt + j, nch);
      if (have_desc) {
        DzChunk& d = sdesc[(k + 2) % 3];
        d.ptr = n_ptr;
        d.aux = 0;
        d.zgroup = n_zg;
        d.n = n_n;
        d.meta = n_meta;
      }
    }
    __syncthreads();
  }
}

// A wait for every vector-memory operation in flight that the compiler sees
// (s_waitcnt with vmcnt 0 and the other counters at their maximum, gfx9
// encoding), so its own bookkeeping knows that nothing is pending after it.
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// One tile of the prefetching tile loop (see rmw_tiles_prefetch): full tile
// k, whose descriptor `ch` the step before read, is computed from `cur`
// (loaded during tile k - 1) while tile k + 1 is loaded into `nxt` (the loads
// go out after the first group, in tile_body). Tile k + 1's descriptor is
// read into `ch1`. Returns whether tile k + 1 is a full tile (its data is
// then in `nxt`); if it is not, the loads read a stand-in of the same size
// (the quantile table), so that every path issues the same loads.
// Descriptor slot (k + 1) % 3 is next written in step k + 2, so the copy read
// here is the one step k + 1 would read; carrying it saves each wave a
// descriptor's LDS reads and its moves to scalar registers per tile. For
// bf16 (ring_tagged), wave 0, which writes the slot, also stores there
// whether the loop can take the tile (kRingTake), so the other waves read
// only the address and the Philox group (one ds_read2_b64, four lane moves;
// no index, n or meta). With these, the bookkeeping below 64 KB of LDS
// (RmwShared) and the wave test taken once (wave0), a thread's VALU
// instructions per tile of the three-way pass went from 459 to 447 for bf16
// (three groups; 2 more on every other step of the unrolled loop) and from
// 430 to 422 for fp16 (four groups). Loading the next tile with buffer loads
// (a descriptor on the scalar unit, 32-bit offsets: no 64-bit address add per
// vector) took 3-4 more off and measured no faster; it is left out. So is
// reading tile k + 1's descriptor from the table with scalar loads in every
// wave (wave 0 has read the entry a step earlier, so they hit the scalar
// cache): 7 fewer per bf16 tile than without take bits (149 per group
// counted), but each tile's start then waits for the scalar loads, and the
// bf16 pass measured 1.4 % faster on one box and 2-3 % slower on two others,
// also with the next index carried from the step before so that those loads
// go out with no LDS read ahead of them.
template <int DT, int MODE>
__device__ __forceinline__ bool rmw_prefetch_step(uint32_t k, const DzChunk& ch, DzChunk& ch1,
                                                  const DzChunk* __restrict__ chunks, uint32_t nchunks,
                                                  const typename RmwTraits<DT, MODE>::E* tab, const DzScalars& sc,
                                                  const TileOffsets<DT, MODE>& to, uint32_t* sidx, DzChunk* sdesc,
                                                  uint32_t* mine, uint32_t ncnt, uint32_t j, const void* dummy,
                                                  bool wave0, const TileRegs<DT, MODE>& cur,
                                                  TileRegs<DT, MODE>& nxt) {
  bool nxt_full;
  if constexpr (ring_tagged(DT)) {
    // The slot's offset is opaque to the compiler, so both fields are read
    // through one address register (one ds_read2_b64), and the take bit is
    // tested on the high word (no 64-bit scalar compare).
    uint32_t slot = (k + 1) % 3 * (uint32_t)sizeof(DzChunk);
    asm("" : "+s"(slot));
    ch1 = uniform_next_chunk(*(const DzChunk*)((const char*)sdesc + slot));
    uint32_t zhi = (uint32_t)(ch1.zgroup >> 32);
    asm("" : "+s"(zhi));  // keeps the test on 32 bits (no 64-bit compare folded back)
    nxt_full = (int32_t)zhi < 0;
    ch1.zgroup = (uint64_t)(zhi & 0x7fffffffu) << 32 | (uint32_t)ch1.zgroup;
  } else {
    const uint32_t c1 = rfl_u32(sidx[(k + 1) % 4]);
    ch1 = uniform_chunk(sdesc[(k + 1) % 3]);
    nxt_full = c1 < nchunks && prefetchable_tile<DT, MODE>(ch1);
  }
  const uint64_t nptr = nxt_full ? ch1.ptr : (uint64_t)(uintptr_t)dummy;
  // wave 0: the ticket of tile k + 3 and the descriptor of tile k + 2
  uint32_t grabbed = 0;
  uint64_t n_ptr = 0, n_zg = 0;
  uint32_t n_n = 0, n_meta = 0;
  bool have_desc = false;
  if (wave0) {  // uniform branch
    if (threadIdx.x == 0) grabbed = atomicAdd(mine, 1u);
    const uint32_t cd = rfl_u32(sidx[(k + 2) % 4]);
    if (cd < nchunks) {
      const DzChunk* src = chunks + cd;
      n_ptr = src->ptr;
      n_zg = src->zgroup;
      n_n = src->n;
      n_meta = src->meta;
      have_desc = true;
      if constexpr (ring_tagged(DT))
        if (prefetchable_tile<DT, MODE>(DzChunk{n_ptr, 0, n_zg, n_n, n_meta})) n_zg |= kRingTake;
    }
  }
  tile_body<DT, MODE, true, true>(ch, to, cur, tab, sc, nptr, &nxt);
  // The ticket is first read here, one straight block after the atomic, so
  // the compiler's wait for it counts the tile's stores and the next tile's
  // loads issued behind it (vmcnt(2 * kVecs)) instead of draining them.
  if (threadIdx.x == 0) {
    sidx[(k + 3) % 4] = (uint32_t)min((uint64_t)grabbed * ncnt + j, (uint64_t)nchunks);
    DzChunk& d = sdesc[(k + 2) % 3];
    if (have_desc) {
      d.ptr = n_ptr;
      d.aux = 0;
      if constexpr (!ring_tagged(DT)) d.zgroup = n_zg;
      d.n = n_n;
      d.meta = n_meta;
    }
    // with the take bit step k + 1 reads; 0 (no take bit) past the table's end
    if constexpr (ring_tagged(DT)) d.zgroup = n_zg;
  }
  lds_barrier();
  return nxt_full;
}

// Tile loop with the next tile's loads in flight during each tile's work,
// over the run of full tiles a workgroup takes first (a table lists its full
// tiles first); the rest of its tiles go through rmw_tiles. Two register
// sets are used in turn (the loop unrolled by two, so no pending registers
// are copied); each step is one straight block whose loads go out at a fixed
// point of it; the ticket is first read in the same straight block as its
// atomic; and the barrier orders LDS only. With those, the compiler's waits for a tile's
// data count the operations behind it (the previous tile's stores and the
// next tile's loads) instead of draining everything in flight.
template <int DT, int MODE>
__device__ __forceinline__ uint32_t rmw_tiles_prefetch(const DzChunk* __restrict__ chunks, uint32_t nchunks,
                                                       const typename RmwTraits<DT, MODE>::E* tab,
                                                       const DzScalars& sc, const TileOffsets<DT, MODE>& to,
                                                       uint32_t* sidx, DzChunk* sdesc, uint32_t* mine, uint32_t ncnt,
                                                       uint32_t j, const void* dummy) {
  const uint32_t c0 = rfl_u32(sidx[0]);
  DzChunk ch0 = uniform_chunk(sdesc[0]);
  if constexpr (ring_tagged(DT)) ch0.zgroup &= ~kRingTake;
  if (!(c0 < nchunks && prefetchable_tile<DT, MODE>(ch0))) return 0;
  // the stand-in must hold a whole tile (a thread's last vector ends at the
  // tile's size)
  static_assert(RmwTraits<DT, MODE>::kChunk <= kDzTabEntries, "the quantile table is a tile's stand-in");
  TileRegs<DT, MODE> a, b;
  DzChunk da = ch0, db;
  const bool wave0 = (rfl_u32(threadIdx.x) >> 6) == 0;
  load_tile_at<DT, MODE>(ch0.ptr, to, a);
  uint32_t k = 0;
  for (;;) {
    if (!rmw_prefetch_step<DT, MODE>(k, da, db, chunks, nchunks, tab, sc, to, sidx, sdesc, mine, ncnt, j, dummy,
                                     wave0, a, b)) {
      k += 1;
      break;
    }
    if (!rmw_prefetch_step<DT, MODE>(k + 1, db, da, chunks, nchunks, tab, sc, to, sidx, sdesc, mine, ncnt, j, dummy,
                                     wave0, b, a)) {
      k += 2;
      break;
    }
    k += 2;
  }
  wait_vm_all();  // the stand-in loads of the last step
  return k;
}

// The RMW kernel's LDS: the tile bookkeeping rings first, so that their
// addresses stay below 64 KB and each wave's reads of them take one address
// register and the DS instructions' 16-bit offset field (with the 128 KB
// table first they took a register per read), then the launch's table.
template <typename E>
struct RmwShared {
  DzChunk sdesc[3];      // descriptors of tiles k .. k + 2
  uint32_t sidx[4];      // indices of tiles k .. k + 3
  E tab[kDzTabEntries];  // the delta table
};

// kPF: run the prefetching tile loop over the workgroup's leading full tiles
// (only where RmwTraits::kPrefetch allows it; the launcher picks it by size).
template <int DT, int MODE, bool kPF>
__global__ void __launch_bounds__(kRmwThreads, kRmwWavesPerEU) rmw_kernel(const DzChunk* __restrict__ chunks,
                                                                          uint32_t nchunks,
                                                                          const void* __restrict__ qtab,
                                                                          DzScalars sc_in, DzScalarPtrs sp,
                                                                          uint32_t* __restrict__ counters) {
  using Tr = RmwTraits<DT, MODE>;
  using E = typename Tr::E;
  __shared__ __attribute__((aligned(16))) RmwShared<E> sh;
  E* const tab = sh.tab;
  uint32_t* const sidx = sh.sidx;
  DzChunk* const sdesc = sh.sdesc;
  const DzScalars sc = resolve_scalars<DT>(sc_in, sp);
  // Counters in use: every one of them must be served by at least one
  // workgroup, or its tiles would never be taken (a small grid uses fewer).
  const uint32_t ncnt = rfl_u32(max(1u, min((uint32_t)kCounters, gridDim.x >> 3)));
  const uint32_t j = rfl_u32((blockIdx.x >> 3) % ncnt);
  uint32_t* mine = counters + j * kCounterStride;
  const uint64_t nch = nchunks;
  // Start-up: lane 0 takes the first three tickets with one atomic, the
  // table's loads are issued behind it, then the first two descriptors are
  // loaded (clamped to a valid index; only tickets below nchunks are used)
  // and the table is written.
  uint32_t t0 = 0;
  if (threadIdx.x == 0) t0 = atomicAdd(mine, 3u);
  TableSlices<DT> qs;
  load_table<DT>(qs, qtab);
  if (threadIdx.x == 0) {
    uint64_t c[3];
    for (int i = 0; i < 3; ++i) {
      c[i] = (uint64_t)(t0 + i) * ncnt + j;
      sidx[i] = (uint32_t)min(c[i], nch);
    }
    if (nch > 0) {
      const DzChunk d0 = chunks[min(c[0], nch - 1)];
      const DzChunk d1 = chunks[min(c[1], nch - 1)];
      sdesc[0] = d0;
      sdesc[1] = d1;
      if constexpr (Tr::kPrefetch && kPF && ring_tagged(DT)) {  // the take bits (kRingTake)
        if (c[0] < nch && prefetchable_tile<DT, MODE>(d0)) sdesc[0].zgroup |= kRingTake;
        if (c[1] < nch && prefetchable_tile<DT, MODE>(d1)) sdesc[1].zgroup |= kRingTake;
      }
    }
  }
  store_table<DT, MODE>(tab, qs, sc);
  const TileOffsets<DT, MODE> to{};
  __syncthreads();
  uint32_t k0 = 0;
  if constexpr (Tr::kPrefetch && kPF)
    k0 = rmw_tiles_prefetch<DT, MODE>(chunks, nchunks, tab, sc, to, sidx, sdesc, mine, ncnt, j, qtab);
  constexpr bool kTagged = Tr::kPrefetch && kPF && ring_tagged(DT);  // the ring may hold take bits
  rmw_tiles<DT, MODE, kTagged>(k0, chunks, nchunks, tab, sc, to, sidx, sdesc, mine, ncnt, j);
  if (threadIdx.x == 0) {
    const uint32_t done = atomicAdd(counters + kDoneSlot * kCounterStride, 1u);
    if (done == gridDim.x - 1) {
      for (int i = 0; i <= kDoneSlot; ++i) atomicExch(counters + i * kCounterStride, 0u);
    }
  }
}

// ---------------------------------------------------------------------------
// Projection kernels over the projected (k/v) tensors, one group per tensor.
//   SUMSQ          partial[c] = sum over chunk of fp32(R_T(theta - theta0))^2
//   APPLY          theta <- R_T(R_T(R_T(theta - theta0) * alpha) + theta0)   trainer.py:428-436
//   REVERSE        theta <- R_T(R_T(R_T(theta - theta0) / alpha) + theta0)   trainer.py:447-451
//   REVERSE_SUMSQ  REVERSE, then partial[c] of the new theta (next norm, trainer.py:455-457)
//   APPLY_F32      theta <- R_T(fp32(R_T(theta - theta0)) * alpha + theta0) with an fp32 alpha:
//                  the first-order path's apply (trainer.py:428-436 with gamma an fp32
//                  Parameter, so v and temp stay fp32 and copy_ rounds once)
// Each chunk is processed by one workgroup; squares and sums in fp64 (exact
// squares of the fp32-widened differences) in a fixed reduction order, so the
// per-chunk partials, and the group sums built from them, are deterministic.
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
  } else if (mode == kProjApplyF32) {
    v = d * alpha;
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

// R_T(a - b) and R_T(a * b) for two packed 16-bit lanes of T (both operands
// in T: the exact difference or product rounded once, which is the
// reference's fp32 op rounded to T).
template <int DT>
__device__ __forceinline__ uint32_t sub_pair(uint32_t a, uint32_t b) {
  if constexpr (DT == DZ_F16) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(dz_half2, a) - __builtin_bit_cast(dz_half2, b));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(dz_bf2, a) - __builtin_bit_cast(dz_bf2, b));
  }
}
template <int DT>
__device__ __forceinline__ uint32_t mul_pair(uint32_t a, uint32_t b) {
  if constexpr (DT == DZ_F16) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(dz_half2, a) * __builtin_bit_cast(dz_half2, b));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(dz_bf2, a) * __builtin_bit_cast(dz_bf2, b));
  }
}

// Sum of squares of the two lanes of a packed 16-bit word, low lane first.
template <int DT>
__device__ __forceinline__ void acc_sq_pair(uint32_t d, double* acc) {
  const double d0 = (double)DT_<DT>::to_f(d & 0xffffu);
  const double d1 = (double)DT_<DT>::to_f(d >> 16);
  *acc += d0 * d0;
  *acc += d1 * d1;
}

// REVERSE's quotient R_T(fp32(d) / alpha) for bf16 T. The reference's fp32
// division rounded to bf16 equals bf16(d * inv), inv = fp32(1 / alpha), for
// every pair of bf16 values d, alpha with inv finite, unless the product is
// nonzero and below the smallest normal fp32 value: checked over all 2^32
// pairs (RN_bf16 of the fp32 quotient is RN_bf16 of the exact quotient, since
// fp32 carries 24 >= 2 * 8 + 2 bits, and for normal operands a bf16 quotient
// is at least 2^-16 of itself away from a bf16 rounding midpoint, where the
// product's error is under 2^-23). Elements outside that range divide. One
// multiply replaces the IEEE division sequence per element.
struct RecipDiv {
  float inv;  // fp32(1 / alpha)
  bool ok;    // inv is finite (alpha is neither 0, infinite nor below 2^-128)
};
__device__ __forceinline__ RecipDiv recip_div(float alpha) {
  const float inv = 1.0f / alpha;
  return RecipDiv{inv, __builtin_isfinite(inv) != 0};
}
__device__ __forceinline__ bool recip_quotient_ok(float q) {
  return !(q != 0.0f && __builtin_fabsf(q) < 0x1p-126f);  // NaN, zero and normal quotients
}

// proj_elem for the two 16-bit elements of a word, in packed arithmetic where
// the reference's op has both operands in T (SUMSQ, APPLY and the subtract /
// add of REVERSE); alpha2 holds alpha in both lanes. APPLY_F32 is not here
// (its fp32 alpha keeps v and the sum in fp32).
template <int DT, int MODE>
__device__ __forceinline__ uint32_t proj_word16(uint32_t th, uint32_t t0, uint32_t alpha2, float alpha,
                                                const RecipDiv& rd, double* acc) {
  const uint32_t d = sub_pair<DT>(th, t0);
  if constexpr (MODE == kProjSumsq) {
    acc_sq_pair<DT>(d, acc);
    return th;
  } else {
    uint32_t v;
    if constexpr (MODE == kProjApply) {
      v = mul_pair<DT>(d, alpha2);
    } else if constexpr (DT == DZ_BF16) {
      const float x0 = bf16_lo_f(d), x1 = bf16_hi_f(d);
      float v0 = x0 * rd.inv, v1 = x1 * rd.inv;
      if (!(rd.ok && recip_quotient_ok(v0) && recip_quotient_ok(v1))) {
        v0 = x0 / alpha;
        v1 = x1 / alpha;
      }
      v = pack_bf16(v0, v1);
    } else {
      const float v0 = DT_<DT>::to_f(d & 0xffffu) / alpha;
      const float v1 = DT_<DT>::to_f(d >> 16) / alpha;
      v = DT_<DT>::from_f(v0) | (DT_<DT>::from_f(v1) << 16);
    }
    const uint32_t nb = add_pair<DT>(v, t0);
    if constexpr (MODE == kProjReverseSumsq) acc_sq_pair<DT>(sub_pair<DT>(nb, t0), acc);
    return nb;
  }
}

__device__ __forceinline__ double block_sum_f64(double x, double* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  const int wid = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wid] = x;
  lds_barrier();
  double t = 0.0;
  if (threadIdx.x == 0) {
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
  }
  return t;
}

// A chunk the vector path takes whole: full size and 16-byte aligned.
template <int DT>
__device__ __forceinline__ bool proj_full_chunk(const DzChunk& ch) {
  return ch.n == (uint32_t)proj_chunk_elems(DT) && (ch.meta & kDzMetaAligned) != 0u;
}

// Vector-memory operations a thread issues for a full chunk: its 16-byte
// loads of theta and theta0, and its stores of theta (none for SUMSQ).
template <int DT, int MODE>
struct ProjChunkOps {
  static constexpr int kVecs = proj_chunk_elems(DT) / (kProjThreads * (16 / (int)sizeof(typename DT_<DT>::S)));
  static constexpr int kAfterTicket = 2 * kVecs + (MODE == kProjSumsq ? 0 : kVecs);
};

// One chunk of a projection launch: the chunk's elements read (theta and
// theta0), updated and written back, and for the SUMSQ modes the chunk's
// partial sum (fixed reduction order) stored at *partial.
template <int DT, int MODE>
__device__ __forceinline__ void proj_chunk(const DzChunk& ch, float alpha, double* partial, double* red) {
  using S = typename DT_<DT>::S;
  constexpr int kES = (int)sizeof(S);
  char* tp = (char*)ch.ptr;
  const char* ap = (const char*)ch.aux;
  double acc = 0.0;
  if (proj_full_chunk<DT>(ch)) {
    constexpr int kVecsPerThread = ProjChunkOps<DT, MODE>::kVecs;
    // alpha in both 16-bit lanes (the ZO modes' alpha is a value of T)
    const uint32_t alpha2 = (kES == 2 && MODE != kProjApplyF32) ? DT_<DT>::from_f(alpha) * 0x10001u : 0u;
    const RecipDiv rd = (DT == DZ_BF16 && (MODE == kProjReverse || MODE == kProjReverseSumsq))
                            ? recip_div(alpha)
                            : RecipDiv{0.0f, false};
    dz_u32x4 vt[kVecsPerThread], va[kVecsPerThread];
#pragma unroll
    for (int u = 0; u < kVecsPerThread; ++u) {
      const size_t off = (size_t)(threadIdx.x + u * kProjThreads) * 16;
      vt[u] = ld_stream(tp + off);
      va[u] = ld_stream(ap + off);
    }
#pragma unroll
    for (int u = 0; u < kVecsPerThread; ++u) {
      dz_u32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kES == 2 && MODE != kProjApplyF32) {
          o[i] = proj_word16<DT, MODE>(vt[u][i], va[u][i], alpha2, alpha, rd, &acc);
        } else if constexpr (kES == 2) {
          uint32_t r0, r1;
          proj_elem<DT>(MODE, vt[u][i] & 0xffffu, va[u][i] & 0xffffu, alpha, &r0, &acc);
          proj_elem<DT>(MODE, vt[u][i] >> 16, va[u][i] >> 16, alpha, &r1, &acc);
          o[i] = (r0 & 0xffffu) | (r1 << 16);
        } else {
          uint32_t r;
          proj_elem<DT>(MODE, vt[u][i], va[u][i], alpha, &r, &acc);
          o[i] = r;
        }
      }
      if constexpr (MODE != kProjSumsq) st_stream(tp + (size_t)(threadIdx.x + u * kProjThreads) * 16, o);
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
    if (threadIdx.x == 0) *partial = t;
  }
}

// alpha of a group: one value of T, or fp32 for APPLY_F32; none for SUMSQ.
template <int DT, int MODE>
__device__ __forceinline__ float group_alpha(const void* __restrict__ alpha_T, uint32_t grp) {
  if constexpr (MODE == kProjSumsq) {
    return 0.0f;
  } else if constexpr (MODE == kProjApplyF32) {
    return ((const float*)alpha_T)[grp];
  } else {
    return DT_<DT>::to_f((uint32_t)((const typename DT_<DT>::S*)alpha_T)[grp]);
  }
}

// Persistent projection kernel: one 1024-thread workgroup per CU takes chunks
// from the table's work counters, as the RMW kernel does (counter j of the K
// in use hands out chunks j, j + K, ...). The groups' alphas are copied to
// LDS once (up to kProjAlphaLds groups; beyond that each chunk reads its
// group's alpha from memory). Wave 0 keeps a pipeline: while chunk k streams,
// lane 0 takes the index of chunk k + 3 and the wave loads the descriptor of
// chunk k + 2 with scalar loads, so no descriptor latency sits between two
// chunks. The last workgroup to finish resets the counters.
template <int DT, int MODE>
__global__ void __launch_bounds__(kProjThreads) proj_kernel(const DzChunk* __restrict__ chunks, uint32_t nchunks,
                                                            uint32_t ngroups, const void* __restrict__ alpha_T,
                                                            double* __restrict__ partials,
                                                            uint32_t* __restrict__ counters) {
  __shared__ double red[kProjThreads / 64];
  __shared__ uint32_t sidx[4];   // chunk indices of k .. k + 3 (ring)
  __shared__ DzChunk sdesc[3];   // descriptors of k .. k + 2
  __shared__ float salpha[MODE == kProjSumsq ? 1 : kProjAlphaLds];
  const bool alpha_in_lds = MODE != kProjSumsq && ngroups <= (uint32_t)kProjAlphaLds;
  if (alpha_in_lds) {
    for (uint32_t g = threadIdx.x; g < ngroups; g += kProjThreads) salpha[g] = group_alpha<DT, MODE>(alpha_T, g);
  }
  const uint32_t ncnt = rfl_u32(max(1u, min((uint32_t)kCounters, gridDim.x >> 3)));
  const uint32_t j = rfl_u32((blockIdx.x >> 3) % ncnt);
  uint32_t* mine = counters + j * kCounterStride;
  const uint64_t nch = nchunks;
  // start-up as in rmw_kernel: three tickets from one atomic, then both
  // descriptors loaded together (clamped to a valid index; only tickets below
  // nchunks are used)
  if (threadIdx.x == 0) {
    const uint32_t t0 = atomicAdd(mine, 3u);
    for (int i = 0; i < 3; ++i) sidx[i] = (uint32_t)min((uint64_t)(t0 + i) * ncnt + j, nch);
    if (nch > 0) {
      const DzChunk d0 = chunks[min((uint64_t)t0 * ncnt + j, nch - 1)];
      const DzChunk d1 = chunks[min((uint64_t)(t0 + 1) * ncnt + j, nch - 1)];
      sdesc[0] = d0;
      sdesc[1] = d1;
    }
  }
  __syncthreads();
  for (uint32_t k = 0;; ++k) {
    const uint32_t c = sidx[k % 4];
    if (c >= nchunks) break;
    const DzChunk ch = uniform_proj_chunk(sdesc[k % 3]);
    const uint32_t grp = ch.meta & kDzMetaGroupMask;
    const float alpha = MODE == kProjSumsq ? 0.0f
                        : alpha_in_lds     ? salpha[grp]
                                           : group_alpha<DT, MODE>(alpha_T, grp);
    uint32_t grabbed = 0;
    uint64_t n_ptr = 0, n_aux = 0;
    uint32_t n_n = 0, n_meta = 0;
    bool have_desc = false;
    if ((rfl_u32(threadIdx.x) >> 6) == 0) {  // wave 0 (uniform branch)
      const uint32_t cd = rfl_u32(sidx[(k + 2) % 4]);
      if (threadIdx.x == 0) grabbed = ticket_take(mine);
      if (cd < nchunks) {
        const DzChunk* src = chunks + cd;
        n_ptr = src->ptr;
        n_aux = src->aux;
        n_n = src->n;
        n_meta = src->meta;
        have_desc = true;
      }
    }
    // lane 0 waits for its ticket behind the chunk's loads and stores (a full
    // chunk issues at least kAfterTicket of them after the ticket; the
    // partial path waits for everything), and the barrier that ends the chunk
    // waits for LDS alone
    if (proj_full_chunk<DT>(ch)) {
      proj_chunk<DT, MODE>(ch, alpha, partials + c, red);
      if (threadIdx.x == 0) ticket_wait<ProjChunkOps<DT, MODE>::kAfterTicket>();
    } else {
      proj_chunk<DT, MODE>(ch, alpha, partials + c, red);
      if (threadIdx.x == 0) ticket_wait<0>();
    }
    if (threadIdx.x == 0) {
      const uint32_t t = ticket_ready(grabbed);
      sidx[(k + 3) % 4] = (uint32_t)min((uint64_t)t * ncnt + j, nch);
      if (have_desc) {
        DzChunk& d = sdesc[(k + 2) % 3];
        d.ptr = n_ptr;
        d.aux = n_aux;
        d.zgroup = 0;
        d.n = n_n;
        d.meta = n_meta;
      }
    }
    lds_barrier();
  }
  if (threadIdx.x == 0) {
    const uint32_t done = atomicAdd(counters + kDoneSlot * kCounterStride, 1u);
    if (done == gridDim.x - 1) {
      for (int i = 0; i <= kDoneSlot; ++i) atomicExch(counters + i * kCounterStride, 0u);
    }
  }
}

// Per-group dot products with other tensors of the same shapes:
//   partial[c] = sum over chunk of fp32(other) * fp32(R_T(theta - theta0))
// (fp64 products of fp32 values are exact; fp64 sums). The gradient of the
// first-order objective with respect to alpha: trainer.py:428-429 under
// autograd gives sum(fp32(grad theta') * fp32(delta)) per projected tensor.
template <int DT>
__global__ void __launch_bounds__(kProjThreads) dot_kernel(const DzChunk* __restrict__ chunks, DzPtrArray other,
                                                           uint32_t group_base, double* __restrict__ partials) {
  using S = typename DT_<DT>::S;
  constexpr int kES = (int)sizeof(S);
  __shared__ double red[kProjThreads / 64];
  const uint32_t c = blockIdx.x;
  const DzChunk ch = chunks[c];
  const uint32_t grp = ch.meta & kDzMetaGroupMask;
  const S* tp = (const S*)ch.ptr;
  const S* ap = (const S*)ch.aux;
  const S* op = (const S*)(other.p[grp - group_base] + ch.zgroup * (uint64_t)kES);
  double acc = 0.0;
  for (uint32_t e = threadIdx.x; e < ch.n; e += kProjThreads) {
    const float d = rt<DT>(DT_<DT>::to_f((uint32_t)tp[e]) - DT_<DT>::to_f((uint32_t)ap[e]));
    acc += (double)DT_<DT>::to_f((uint32_t)op[e]) * (double)d;
  }
  const double t = block_sum_f64(acc, red);
  if (threadIdx.x == 0) partials[c] = t;
}

// Per-group reduction of chunk partials, in chunk order. With take_sqrt:
// norm = R_T(sqrt_f32(fp32(sum)))  (torch.norm: fp32 accumulate, fp32 sqrt, cast to T);
// without: the fp32 / T outputs hold the rounded sum itself.
template <int DT>
__global__ void __launch_bounds__(kProjThreads) finalize_kernel(const double* __restrict__ partials,
                                                                const uint32_t* __restrict__ gbegin,
                                                                double* __restrict__ sumsq,
                                                                float* __restrict__ norm_f32,
                                                                void* __restrict__ norm_T, bool take_sqrt) {
  using S = typename DT_<DT>::S;
  __shared__ double red[kProjThreads / 64];
  const uint32_t g = blockIdx.x;
  const uint32_t b = gbegin[g], e = gbegin[g + 1];
  double x = 0.0;
  for (uint32_t i = b + threadIdx.x; i < e; i += kProjThreads) x += partials[i];
  const double t = block_sum_f64(x, red);
  if (threadIdx.x == 0) {
    // correctly rounded fp32 sqrt of the fp32 sum (a double sqrt rounds once more, exactly)
    const float n = take_sqrt ? (float)sqrt((double)(float)t) : (float)t;
    if (sumsq) sumsq[g] = t;
    if (norm_f32) norm_f32[g] = n;
    if (norm_T) ((S*)norm_T)[g] = (S)DT_<DT>::from_f(n);
  }
}

// Chunk descriptors of a projection launch planned on the device (the
// table-free norm pass): block g writes group g's chunks, split as
// dz_table_create splits them (proj_chunk_elems(dtype) elements, the last one shorter;
// aligned when theta and theta0 are 16-byte aligned), and its first chunk
// index; the last batch also writes the end index of the last group. The
// first batch zeroes the work counters the projection kernel takes chunks
// from.
__global__ void __launch_bounds__(256) static_plan_kernel(StaticPlanBatch b, DzChunk* __restrict__ chunks,
                                                          uint32_t* __restrict__ group_begin,
                                                          uint32_t* __restrict__ counters) {
  const uint32_t g = blockIdx.x;
  if (b.first && g == 0) {
    for (int i = threadIdx.x; i < kCounterWords; i += blockDim.x) counters[i] = 0u;
  }
  if (g >= b.ngroups) return;
  const uint32_t gi = b.group_base + g;
  const uint64_t p = b.ptr[g], a = b.anchor[g];
  const int64_t ne = b.numel[g];
  const uint32_t meta = gi | ((p % 16 == 0 && a % 16 == 0) ? kDzMetaAligned : 0u);
  const int64_t cn = b.chunk_elems;
  const uint32_t nch = (uint32_t)((ne + cn - 1) / cn);
  for (uint32_t k = threadIdx.x; k < nch; k += blockDim.x) {
    const uint64_t s = (uint64_t)k * (uint64_t)cn;
    DzChunk c;
    c.ptr = p + s * (uint64_t)b.elem_size;
    c.aux = a + s * (uint64_t)b.elem_size;
    c.zgroup = s;
    c.n = (uint32_t)min(cn, ne - (int64_t)s);
    c.meta = meta;
    chunks[b.chunk_begin[g] + k] = c;
  }
  if (threadIdx.x == 0) {
    group_begin[gi] = b.chunk_begin[g];
    if (gi + 1 == b.total_groups) group_begin[b.total_groups] = b.total_chunks;
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
// With timing events given (LaunchEvents), a launch goes through
// hipExtLaunchKernel, which records them when the kernel starts and ends.
// ---------------------------------------------------------------------------
#define DZ_LAUNCH(kernel, grid, block, st, ev, ...)                                              \
  do {                                                                                          \
    if ((ev).start || (ev).stop) {                                                              \
      hipExtLaunchKernelGGL(kernel, grid, block, 0, st, (ev).start, (ev).stop, 0, __VA_ARGS__); \
    } else {                                                                                    \
      hipLaunchKernelGGL(kernel, grid, block, 0, st, __VA_ARGS__);                              \
    }                                                                                           \
  } while (0)

template <int DT>
static hipError_t launch_rmw_dt(int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t grid,
                                const void* tab, const DzScalars& s, const DzScalarPtrs& p,
                                uint32_t* counters, bool prefetch, hipStream_t st, const LaunchEvents& ev) {
  switch (mode) {
    case kModePerturb:
      DZ_LAUNCH((rmw_kernel<DT, kModePerturb, false>), dim3(grid), dim3(kRmwThreads), st, ev,
                         chunks, nchunks, tab, s, p, counters);
      break;
    case kModeUpdate:
      DZ_LAUNCH((rmw_kernel<DT, kModeUpdate, false>), dim3(grid), dim3(kRmwThreads), st, ev,
                         chunks, nchunks, tab, s, p, counters);
      break;
    case kModeRestoreUpdate:
      DZ_LAUNCH((rmw_kernel<DT, kModeRestoreUpdate, false>), dim3(grid), dim3(kRmwThreads),
                         st, ev, chunks, nchunks, tab, s, p, counters);
      break;
    case kModeRestoreUpdatePerturb:
      // the caller asks for the prefetching loop on long launches (the table's prefetch_min_tiles)
      if (RmwTraits<DT, kModeRestoreUpdatePerturb>::kPrefetch && prefetch) {
        DZ_LAUNCH((rmw_kernel<DT, kModeRestoreUpdatePerturb, true>), dim3(grid), dim3(kRmwThreads),
                           st, ev, chunks, nchunks, tab, s, p, counters);
      } else {
        DZ_LAUNCH((rmw_kernel<DT, kModeRestoreUpdatePerturb, false>), dim3(grid), dim3(kRmwThreads),
                           st, ev, chunks, nchunks, tab, s, p, counters);
      }
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rmw(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t grid,
                      const void* tab, const DzScalars& s, const DzScalarPtrs& p, uint32_t* counters,
                      bool prefetch, hipStream_t st, const LaunchEvents& ev) {
  switch (dtype) {
    case DZ_F32:
      return launch_rmw_dt<DZ_F32>(mode, chunks, nchunks, grid, tab, s, p, counters, prefetch, st, ev);
    case DZ_F16:
      return launch_rmw_dt<DZ_F16>(mode, chunks, nchunks, grid, tab, s, p, counters, prefetch, st, ev);
    case DZ_BF16:
      return launch_rmw_dt<DZ_BF16>(mode, chunks, nchunks, grid, tab, s, p, counters, prefetch, st, ev);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
static hipError_t launch_proj_dt(int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t ngroups,
                                 uint32_t grid, const void* alpha, double* partials, uint32_t* counters,
                                 hipStream_t st, const LaunchEvents& ev) {
  switch (mode) {
    case kProjSumsq:
      DZ_LAUNCH((proj_kernel<DT, kProjSumsq>), dim3(grid), dim3(kProjThreads), st, ev, chunks, nchunks,
                         ngroups, alpha, partials, counters);
      break;
    case kProjApply:
      DZ_LAUNCH((proj_kernel<DT, kProjApply>), dim3(grid), dim3(kProjThreads), st, ev, chunks, nchunks,
                         ngroups, alpha, partials, counters);
      break;
    case kProjReverse:
      DZ_LAUNCH((proj_kernel<DT, kProjReverse>), dim3(grid), dim3(kProjThreads), st, ev, chunks, nchunks,
                         ngroups, alpha, partials, counters);
      break;
    case kProjReverseSumsq:
      DZ_LAUNCH((proj_kernel<DT, kProjReverseSumsq>), dim3(grid), dim3(kProjThreads), st, ev, chunks,
                         nchunks, ngroups, alpha, partials, counters);
      break;
    case kProjApplyF32:
      DZ_LAUNCH((proj_kernel<DT, kProjApplyF32>), dim3(grid), dim3(kProjThreads), st, ev, chunks, nchunks,
                         ngroups, alpha, partials, counters);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_proj(int dtype, int mode, const DzChunk* chunks, uint32_t nchunks, uint32_t ngroups,
                       uint32_t grid, const void* alpha, double* partials, uint32_t* counters, hipStream_t st,
                       const LaunchEvents& ev) {
  switch (dtype) {
    case DZ_F32:
      return launch_proj_dt<DZ_F32>(mode, chunks, nchunks, ngroups, grid, alpha, partials, counters, st, ev);
    case DZ_F16:
      return launch_proj_dt<DZ_F16>(mode, chunks, nchunks, ngroups, grid, alpha, partials, counters, st, ev);
    case DZ_BF16:
      return launch_proj_dt<DZ_BF16>(mode, chunks, nchunks, ngroups, grid, alpha, partials, counters, st, ev);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dot(int dtype, const DzChunk* chunks, uint32_t nchunks, const DzPtrArray& other,
                      uint32_t group_base, double* partials, hipStream_t st, const LaunchEvents& ev) {
  switch (dtype) {
    case DZ_F32:
      DZ_LAUNCH((dot_kernel<DZ_F32>), dim3(nchunks), dim3(kProjThreads), st, ev, chunks, other,
                         group_base, partials);
      break;
    case DZ_F16:
      DZ_LAUNCH((dot_kernel<DZ_F16>), dim3(nchunks), dim3(kProjThreads), st, ev, chunks, other,
                         group_base, partials);
      break;
    case DZ_BF16:
      DZ_LAUNCH((dot_kernel<DZ_BF16>), dim3(nchunks), dim3(kProjThreads), st, ev, chunks, other,
                         group_base, partials);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_finalize(int dtype, const double* partials, const uint32_t* gbegin, uint32_t ngroups,
                           double* sumsq, float* norm_f32, void* norm_T, bool take_sqrt, hipStream_t st,
                           const LaunchEvents& ev) {
  switch (dtype) {
    case DZ_F32:
      DZ_LAUNCH((finalize_kernel<DZ_F32>), dim3(ngroups), dim3(kProjThreads), st, ev,
                         partials, gbegin, sumsq, norm_f32, norm_T, take_sqrt);
      break;
    case DZ_F16:
      DZ_LAUNCH((finalize_kernel<DZ_F16>), dim3(ngroups), dim3(kProjThreads), st, ev,
                         partials, gbegin, sumsq, norm_f32, norm_T, take_sqrt);
      break;
    case DZ_BF16:
      DZ_LAUNCH((finalize_kernel<DZ_BF16>), dim3(ngroups), dim3(kProjThreads), st, ev,
                         partials, gbegin, sumsq, norm_f32, norm_T, take_sqrt);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_static_plan(const StaticPlanBatch& b, DzChunk* chunks, uint32_t* group_begin, uint32_t* counters,
                              hipStream_t st) {
  hipLaunchKernelGGL(static_plan_kernel, dim3(b.ngroups ? b.ngroups : 1), dim3(256), 0, st, b, chunks, group_begin,
                     counters);
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

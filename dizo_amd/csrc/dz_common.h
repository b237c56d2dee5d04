// Shared host/device definitions for the DiZO zeroth-order step kernels.
//
// Contents:
//   * dtype codes used across the C ABI,
//   * the chunk descriptor that the multi-tensor kernels walk,
//   * Philox4x32-7, the counter-based generator that regenerates z in registers,
//   * the z definition: z(seed, e) for global element index e.
//
// Philox4x32-R follows Salmon, Moraes, Dror and Shaw, "Parallel Random Numbers:
// As Easy as 1, 2, 3" (SC'11): four 32-bit counter words, a two-word key, R
// rounds of two 32x32->64 multiplies by 0xD2511F53 / 0xCD9E8D57, with the key
// bumped by the Weyl constants 0x9E3779B9 / 0xBB67AE85 between rounds. z uses
// R = 7, the fewest rounds the paper found Crush-resistant for Philox4x32 (it
// passes TestU01's BigCrush; the paper's default of 10 keeps three rounds in
// hand). Each round costs two 32x32->64 products and two three-way xors per
// block, and the fused restore + update + next perturbation pass draws two
// blocks per 8 elements, so the round count sets most of its ALU work.
//
// z definition (replaces torch.normal at trainer.py:1441 and :1607):
//   key  = (seed mod 2^32, seed >> 32)
//   e    = global element index (tensors laid end to end, each tensor starting
//          at a multiple of 8, in named_parameters_to_optim order)
//   w    = Philox4x32-7(counter = (stream, q mod 2^32, 0, q >> 32), key), q = e >> 3
//   h    = 16-bit field (e & 7) of w (field j = bits 16*(j&1).. of word j>>1)
//   z    = (h & 0x8000 ? -1 : +1) * Q_T[h & 0x7fff]
//   Q_T[i] = RNE_T( Phi^{-1}( 1/2 + (i + 1/2) / 65536 ) )
// i.e. a sign bit and a 15-bit quantile index per element: eight normals per
// Philox call, each already exact in the parameter dtype T.
//
// Counter layout. A round multiplies counter words 0 and 2 and xors words 1
// and 3 into the products' high halves. The word that differs between the
// lanes of a wave (q mod 2^32) sits in word 1, so it enters by an xor in
// round 0 and is first multiplied in round 1; the stream, the zero word and
// the high word of q (the same across a tile of one tensor) are uniform. The
// kernels then run round 0, the products of one word in rounds 1 and 2, and
// the xors of their results on the scalar unit: ten vector multiplies per
// block against twelve with q in word 0. The three-way restore + update +
// next perturbation pass draws two blocks per 8 elements, so that is four
// fewer per group.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>
#define DZ_HD __host__ __device__ __forceinline__
#else
#define DZ_HD static inline
#endif

#if defined(__HIPCC__) || defined(__HIP__)
// Opaque identity: the value must exist as a plain fp32 register here. Placed
// between an fp32 product and its conversion to a 16-bit type, it keeps the
// backend from folding the two into one mixed-precision FMA (which rounds the
// exact product once instead of twice, as PyTorch does).
__device__ __forceinline__ float dz_opq(float x) {
  asm("" : "+v"(x));
  return x;
}
#endif

enum DzDtype : int32_t { DZ_F32 = 0, DZ_F16 = 1, DZ_BF16 = 2 };

// Stream ids of the Philox counter word 2.
constexpr uint32_t kDzStreamParam = 0;  // z of the parameter perturbation / update
constexpr uint32_t kDzStreamGamma = 1;  // z of the DiZO gamma perturbation (trainer.py:554)
constexpr uint32_t kDzStreamInit = 2;   // synthetic weight initialisation

constexpr int kDzTabEntries = 32768;  // quantile table entries (15-bit index)

// One unit of work of a multi-tensor kernel: up to `chunk_elems` consecutive
// elements of one tensor. Built on the host, uploaded once per table.
struct DzChunk {
  uint64_t ptr;     // byte address of the chunk's first element (theta)
  uint64_t aux;     // byte address of the matching anchor element (theta0), or 0
  uint64_t zgroup;  // ZO tables: Philox counter q of the chunk's first element (e / 8);
                    // projection tables: element offset of the chunk in its tensor
  uint32_t n;       // number of elements in the chunk
  uint32_t meta;    // bits 0..23: tensor/group index; bit 31: all pointers 16-byte aligned
};
static_assert(sizeof(DzChunk) == 32, "DzChunk must stay 32 bytes");

constexpr uint32_t kDzMetaAligned = 0x80000000u;
constexpr uint32_t kDzMetaGroupMask = 0x00ffffffu;

struct DzU4 {
  uint32_t x, y, z, w;
};

DZ_HD void dz_mulhilo32(uint32_t a, uint32_t b, uint32_t* lo, uint32_t* hi) {
  const uint64_t p = (uint64_t)a * (uint64_t)b;
  *lo = (uint32_t)p;
  *hi = (uint32_t)(p >> 32);
}

// Philox4x32 with R rounds (z uses R = kDzPhiloxRounds).
template <int R>
DZ_HD DzU4 dz_philox4x32(DzU4 c, uint32_t k0, uint32_t k1) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
#endif
  for (int r = 0; r < R; ++r) {
    uint32_t lo0, hi0, lo1, hi1;
    dz_mulhilo32(0xD2511F53u, c.x, &lo0, &hi0);
    dz_mulhilo32(0xCD9E8D57u, c.z, &lo1, &hi1);
    DzU4 n;
#if defined(__HIP_DEVICE_COMPILE__)
    if (r < 3) {
      // Plain xors: with the z counter layout some of these operands are
      // uniform (all of them for n.x in round 1 and n.z in round 0), and a
      // uniform result stays on the scalar unit, with the next round's
      // product of it (the bitop3 builtin is vector-only).
      n.x = hi1 ^ c.y ^ k0;
      n.z = hi0 ^ c.w ^ k1;
    } else {
      // gfx950 three-input bitwise op; truth table 0x96 is a ^ b ^ c
      n.x = __builtin_amdgcn_bitop3_b32(hi1, c.y, k0, 0x96);
      n.z = __builtin_amdgcn_bitop3_b32(hi0, c.w, k1, 0x96);
    }
#else
    n.x = hi1 ^ c.y ^ k0;
    n.z = hi0 ^ c.w ^ k1;
#endif
    n.y = lo1;
    n.w = lo0;
    c = n;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// Rounds of the Philox that defines z (part of the z definition: the oracle's
// rng.ROUNDS must match).
constexpr int kDzPhiloxRounds = 7;

// The block of counter q = q_hi * 2^32 + q_lo, with the two words passed
// apart (a caller whose q_hi is uniform across a wave keeps it scalar).
// Counter words (stream, q_lo, 0, q_hi): see "Counter layout" above.
DZ_HD DzU4 dz_philox_counter(uint64_t seed, uint32_t stream, uint32_t q_lo, uint32_t q_hi) {
  DzU4 c;
  c.x = stream;
  c.y = q_lo;
  c.z = 0u;
  c.w = q_hi;
  return dz_philox4x32<kDzPhiloxRounds>(c, (uint32_t)seed, (uint32_t)(seed >> 32));
}

DZ_HD DzU4 dz_philox_group(uint64_t seed, uint32_t stream, uint64_t q) {
  return dz_philox_counter(seed, stream, (uint32_t)q, (uint32_t)(q >> 32));
}

// 16-bit field j (0..7) of a Philox output block.
DZ_HD uint32_t dz_field16(const DzU4& w, int j) {
  const uint32_t word = (j >> 1) == 0 ? w.x : (j >> 1) == 1 ? w.y : (j >> 1) == 2 ? w.z : w.w;
  return (word >> (16 * (j & 1))) & 0xffffu;
}

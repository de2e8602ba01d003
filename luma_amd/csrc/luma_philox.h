// Philox4x32-10 counter-based generator (Salmon, Moraes, Dror, Shaw,
// "Parallel Random Numbers: As Easy as 1, 2, 3", SC'11), host and device.
//
// One block maps a 128-bit counter and a 64-bit key to 128 random bits with
// ten rounds of two 32x32->64 multiplies; the key is bumped by the Weyl
// constants between rounds.
//
// How the LUMA step uses it (the uniform stream of one (param, step)):
//   key      = seed = ((t << 32) | 2*param_id) ^ base_seed  (the reference's
//              per-step seed, functional.py:99-106), split lo/hi.
//   element e gets two 24-bit uniforms u_m(e), u_w(e) in [0, 1); with
//   j = e & 7 and the three blocks of its group of 8 elements,
//     T_m = ctr (B + (e >> 3), 0, r),  L = ctr (B + (e >> 3), 1, r),
//     T_w = ctr (B + (e >> 3), 2, r):
//     u_m: high 16 bits -- half j of T_m;  low 8 bits -- byte 2j of L
//     u_w: high 16 bits -- half j of T_w;  low 8 bits -- byte 2j + 1 of L
//   (counter words: c0 = lo32(index), c1 = hi32(index), c2 = stream, c3 = r).
// B = o >> 3 and r = o & 7 come from the tensor's element offset o: the
// index of its element 0 in the whole parameter when the tensor is one shard
// of it (0 otherwise).  A shard whose offset is a multiple of 8 therefore
// draws exactly the uniforms of the same elements of the unsharded
// parameter; shards with another offset draw from the disjoint counter
// space r != 0, and two shards of one parameter never share a block (their
// element ranges are disjoint, so their block ranges are too).
// The split lets the fast path decide almost every rounding from the two
// 16-bit blocks and fetch the low bits only for the rare elements whose
// decision depends on them.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define LUMA_PHILOX_FN __host__ __device__ __forceinline__
#else
#define LUMA_PHILOX_FN static inline
#endif

namespace luma {

constexpr uint32_t kPhiloxM0 = 0xD2511F53u;
constexpr uint32_t kPhiloxM1 = 0xCD9E8D57u;
constexpr uint32_t kPhiloxW0 = 0x9E3779B9u;
constexpr uint32_t kPhiloxW1 = 0xBB67AE85u;

struct U4 {
  uint32_t x, y, z, w;
};

LUMA_PHILOX_FN void philox_round(uint32_t &c0, uint32_t &c1, uint32_t &c2, uint32_t &c3, uint32_t k0,
                          uint32_t k1) {
  const uint64_t p0 = (uint64_t)kPhiloxM0 * c0;
  const uint64_t p1 = (uint64_t)kPhiloxM1 * c2;
  const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
  const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
  const uint32_t n0 = hi1 ^ c1 ^ k0;
  const uint32_t n2 = hi0 ^ c3 ^ k1;
  c0 = n0;
  c1 = lo1;
  c2 = n2;
  c3 = lo0;
}

// Ten rounds; round r uses key (k0 + r*W0, k1 + r*W1).
LUMA_PHILOX_FN U4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                         uint32_t k1) {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
#endif
  for (int r = 0; r < 10; ++r) {
    philox_round(c0, c1, c2, c3, k0, k1);
    k0 += kPhiloxW0;
    k1 += kPhiloxW1;
  }
  U4 o;
  o.x = c0;
  o.y = c1;
  o.z = c2;
  o.w = c3;
  return o;
}

#if defined(__HIPCC__)
// Device variant with the multipliers passed in (callers keep them, and the
// key, in VGPRs; see in_vgpr in luma_step.hip).  Each three-way xor is one
// v_bitop3_b32 (truth table 0x96, gfx950) instead of two v_xor_b32: the
// compiler does not form it from a ^ b ^ c by itself.
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ U4 philox4x32_10_v(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                              uint32_t k0, uint32_t k1, uint32_t m0,
                                              uint32_t m1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)m0 * c0;
    const uint64_t p1 = (uint64_t)m1 * c2;
    const uint32_t n0 = xor3((uint32_t)(p1 >> 32), c1, k0);
    const uint32_t n2 = xor3((uint32_t)(p0 >> 32), c3, k1);
    c0 = n0;
    c1 = (uint32_t)p1;
    c2 = n2;
    c3 = (uint32_t)p0;
    k0 += kPhiloxW0;
    k1 += kPhiloxW1;
  }
  return U4{c0, c1, c2, c3};
}
#endif

// Where a tensor's blocks start: B = offset >> 3 and r = offset & 7 of its
// element offset (see the header comment).
struct PhiloxBase {
  uint64_t blk;
  uint32_t rot;
};

LUMA_PHILOX_FN PhiloxBase philox_base(int64_t elem_offset) {
  PhiloxBase b;
  b.blk = (uint64_t)elem_offset >> 3;
  b.rot = (uint32_t)elem_offset & 7u;
  return b;
}

// Block `stream` of element e's group of 8 (kBlockTopM, kBlockLow, kBlockTopW).
constexpr uint32_t kBlockTopM = 0u, kBlockLow = 1u, kBlockTopW = 2u;

LUMA_PHILOX_FN U4 philox_block(uint64_t e, PhiloxBase o, uint32_t stream, uint32_t k0,
                               uint32_t k1) {
  const uint64_t b = o.blk + (e >> 3);
  return philox4x32_10((uint32_t)b, (uint32_t)(b >> 32), stream, o.rot, k0, k1);
}

LUMA_PHILOX_FN uint32_t u4_word(const U4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Byte i (0..15) of a block, little-endian across x, y, z, w.
LUMA_PHILOX_FN uint32_t u4_byte(const U4 &v, int i) { return (u4_word(v, i >> 2) >> (8 * (i & 3))) & 0xFFu; }

// 16-bit half i (0..7) of a block.
LUMA_PHILOX_FN uint32_t u4_half(const U4 &v, int i) { return (u4_word(v, i >> 1) >> (16 * (i & 1))) & 0xFFFFu; }

// The two 24-bit integers (u * 2^24) of element e, from its group's blocks.
LUMA_PHILOX_FN void philox_uniform_bits(const U4 &top_m, const U4 &top_w, const U4 &low, uint64_t e,
                                        uint32_t &bits_m, uint32_t &bits_w) {
  const int j = (int)(e & 7);
  bits_m = (u4_half(top_m, j) << 8) | u4_byte(low, 2 * j);
  bits_w = (u4_half(top_w, j) << 8) | u4_byte(low, 2 * j + 1);
}

}  // namespace luma

// Shared host/device pieces of the bloom retrieval path: index geometry, the
// murmur hash split into its seed-independent and seed-dependent halves, and
// exact 64-bit modulo by a runtime divisor.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define ST_HD __host__ __device__ __forceinline__
#else
#define ST_HD inline
#endif

// The kernels are written for gfx950 (MI355X): 160 KB of LDS per workgroup
// (the search tile, the wide-bundle slice, kmean_ann's staging), wave64.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "silvertorch_amd device code is built for gfx950 only"
#endif

namespace st {

constexpr int64_t kBitsPerColumn = 64;
constexpr int64_t kColumnsPerBundle = 32;
constexpr int64_t kDocsPerBundle = kBitsPerColumn * kColumnsPerBundle;
constexpr int64_t kMaxSearchK = 10;  // MAX_K_V2, bloom_index_util.h:45
constexpr int64_t kMaxBuildK = 64;   // MAX_K, bloom_index_util.h:39

// Plan operator codes of the encoded query plans (bloom_index_util.h:48-55).
enum PlanOp : uint8_t {
  kOpAnd = 1,
  kOpOr = 2,
  kOpNot = 3,
  kOpTerm = 4,
  kOpEmpty = 5,
};

ST_HD uint64_t rotl64(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }

ST_HD uint64_t fmix64(uint64_t h) {
  h ^= h >> 33;
  h *= 0xff51afd7ed558ccdULL;
  h ^= h >> 33;
  h *= 0xc4ceb9fe1a85ec53ULL;
  h ^= h >> 33;
  return h;
}

// MurmurHash3_x64_128 on the 16-byte little-endian key x||y (one full block,
// no tail, length 16), both lanes seeded with `seed`, folded to h1 ^ h2.
// Same function as murmur_hash3_2x64 (bloom_index_util.cuh:59-106).  The
// block mixing of x and y does not depend on the seed, so callers that hash
// one key under many seeds compute mix_x / mix_y once and call
// murmur_finish per seed.
ST_HD uint64_t murmur_mix_x(uint64_t x) {
  return rotl64(x * 0x87c37b91114253d5ULL, 31) * 0x4cf5ad432745937fULL;
}
ST_HD uint64_t murmur_mix_y(uint64_t y) {
  return rotl64(y * 0x4cf5ad432745937fULL, 33) * 0x87c37b91114253d5ULL;
}
ST_HD uint64_t murmur_finish(uint64_t mx, uint64_t my, uint64_t seed) {
  uint64_t h1 = rotl64(seed ^ mx, 27) + seed;
  h1 = h1 * 5 + 0x52dce729ULL;
  uint64_t h2 = rotl64(seed ^ my, 31) + h1;
  h2 = h2 * 5 + 0x38495ab5ULL;
  h1 ^= 16;
  h2 ^= 16;
  h1 += h2;
  h2 += h1;
  h1 = fmix64(h1);
  h2 = fmix64(h2);
  h1 += h2;
  h2 += h1;
  return h1 ^ h2;
}
ST_HD uint64_t murmur_pair(uint64_t x, uint64_t y, uint64_t seed) {
  return murmur_finish(murmur_mix_x(x), murmur_mix_y(y), seed);
}

// murmur_finish for one key under many small seeds: the seed enters the
// rotations only through seed ^ mx and seed ^ my, and for seed < 2^27
// rotl(seed ^ m, r) = rotl(m, r) ^ (seed << r) (r = 27, 31), so the
// rotations of mx and my are taken once per key (rx = rotl(mx, 27),
// ry = rotl(my, 31)).  Equal to murmur_finish(mx, my, seed) for those seeds.
ST_HD uint64_t murmur_finish_rot(uint64_t rx, uint64_t ry, uint64_t seed) {
  uint64_t h1 = (rx ^ (seed << 27)) + seed;
  h1 = h1 * 5 + 0x52dce729ULL;
  uint64_t h2 = (ry ^ (seed << 31)) + h1;
  h2 = h2 * 5 + 0x38495ab5ULL;
  h1 ^= 16;
  h2 ^= 16;
  h1 += h2;
  h2 += h1;
  h1 = fmix64(h1);
  h2 = fmix64(h2);
  h1 += h2;
  h2 += h1;
  return h1 ^ h2;
}

ST_HD uint64_t mulhi64(uint64_t a, uint64_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul64hi(a, b);
#else
  return static_cast<uint64_t>((static_cast<unsigned __int128>(a) * b) >> 64);
#endif
}

// n % d for a fixed divisor d >= 1, without a 64-bit divide per call.
// magic = floor((2^64 - 1) / d), so q = mulhi(n, magic) satisfies
// floor(n/d) - 2 <= q <= floor(n/d); at most two corrections follow.
struct FastMod64 {
  uint64_t d;
  uint64_t magic;
};

ST_HD FastMod64 make_fastmod(uint64_t d) {
  FastMod64 f;
  f.d = d;
  f.magic = d ? (~0ULL) / d : 0;
  return f;
}

ST_HD uint64_t fast_mod(uint64_t n, const FastMod64& f) {
  uint64_t q = mulhi64(n, f.magic);
  uint64_t r = n - q * f.d;
  if (r >= f.d) r -= f.d;
  if (r >= f.d) r -= f.d;
  return r;
}

// fast_mod for divisors below 2^30: n - q * d lies in [0, 3d) < 2^32, so it
// equals its low 32 bits, and those are n_lo - q_lo * d (mod 2^32).
ST_HD uint32_t fast_mod_small(uint64_t n, const FastMod64& f) {
  const uint64_t q = mulhi64(n, f.magic);
  const uint32_t d = static_cast<uint32_t>(f.d);
  uint32_t r = static_cast<uint32_t>(n) - static_cast<uint32_t>(q) * d;
  if (r >= d) r -= d;
  if (r >= d) r -= d;
  return r;
}

#if defined(__HIPCC__)
// make_fastmod in device code without a 64-bit divide for divisors below
// 2^32, from 32-bit divides only:
// (2^64-1)/d = ((2^32-1)/d) * 2^32 + (((2^32-1) % d) * 2^32 + 2^32-1) / d.
__device__ __forceinline__ FastMod64 make_fastmod_dev(uint64_t d) {
  if (d == 0 || (d >> 32)) return make_fastmod(d);
  const uint32_t d32 = static_cast<uint32_t>(d);
  const uint32_t qh = 0xFFFFFFFFu / d32;
  const uint32_t rh = 0xFFFFFFFFu % d32;
  const uint64_t n = (static_cast<uint64_t>(rh) << 32) | 0xFFFFFFFFull;  // < d * 2^32
  uint64_t ql = static_cast<uint64_t>(static_cast<double>(n) / static_cast<double>(d32));
  // the double quotient is within one of the true one; fix it exactly
  while (ql * d32 > n) --ql;
  while (n - ql * d32 >= d32) ++ql;
  FastMod64 f;
  f.d = d;
  f.magic = (static_cast<uint64_t>(qh) << 32) + ql;
  return f;
}
#endif

}  // namespace st

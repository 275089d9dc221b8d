// hash.hip -- FarmHash Fingerprint64 on gfx950 and the hash-bucket embedding
// ops built on it.
//
// Fingerprint64 is farmhashna::Hash64 from google/farmhash (the
// @farmhash_archive TensorFlow 2.15 links), which ANNC reaches through
// util::Fingerprint64 / tensorflow::Fingerprint64
// (python/tensorflow/kernels/fused_embedding_with_hash_bucket.cc:63,
//  fused_dnn_embedding_with_hash_bucket.cc:30, fused_sparse_embedding.cc:36).
// Two device formulations:
//   * fp64_bytes: any string in global memory (byte loads; all length
//     branches including the 64-byte block loop);
//   * fp64_decimal: the decimal text of an int64 (AsString semantics, the
//     op pattern replaced at python/annc/optimize/rec_embedding.py:549-557)
//     built directly in three 64-bit registers -- at most 20 bytes, so only
//     the 0-16 and 17-32 byte branches exist -- with no memory traffic.
// CDNA has no 64x64-bit multiplier; the 64-bit products compile to 32-bit
// v_mul_lo/v_mul_hi sequences, and `% num_buckets` uses a precomputed
// invariant-divisor reciprocal instead of a 64-bit division loop.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "scan_sort.h"
#include "embedding_impl.h"

namespace annc {

U64Divisor make_divisor(uint64_t d) {
  U64Divisor r{d, 0, -1};
  if (d <= 1) return r;
  const int l = 64 - __builtin_clzll(d - 1);  // ceil(log2 d), 1..64
  const uint64_t two_l_minus_d = (l == 64 ? 0ull : (1ull << l)) - d;  // mod 2^64
  const unsigned __int128 num = static_cast<unsigned __int128>(two_l_minus_d) << 64;
  r.magic = static_cast<uint64_t>(num / d) + 1;
  r.shift = l - 1;
  return r;
}

namespace {

constexpr uint64_t kC0 = 0xc3a5c85c97cb3127ULL;
constexpr uint64_t kC1 = 0xb492b66fbe98f273ULL;
constexpr uint64_t kC2 = 0x9ae16a3b2f90404fULL;
constexpr int kThreads = 256;
constexpr int kMaxFields = 64;

__device__ __forceinline__ uint64_t rotr(uint64_t v, int s) { return (v >> s) | (v << (64 - s)); }
__device__ __forceinline__ uint64_t smix(uint64_t v) { return v ^ (v >> 47); }

__device__ __forceinline__ uint64_t mix16(uint64_t u, uint64_t v, uint64_t mul) {
  uint64_t a = (u ^ v) * mul;
  a ^= a >> 47;
  uint64_t b = (v ^ a) * mul;
  b ^= b >> 47;
  return b * mul;
}

__device__ __forceinline__ uint64_t mod_invariant(uint64_t n, const U64Divisor& dv) {
  if (dv.shift < 0) return 0;  // d == 1
  const uint64_t t1 = __umul64hi(dv.magic, n);
  const uint64_t q = (t1 + ((n - t1) >> 1)) >> dv.shift;
  return n - q * dv.d;
}

// ---------------------------------------------------------------------------
// Strings in memory.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t le64(const unsigned char* p) {
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) r |= static_cast<uint64_t>(p[i]) << (8 * i);
  return r;
}
__device__ __forceinline__ uint64_t le32(const unsigned char* p) {
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) r |= static_cast<uint64_t>(p[i]) << (8 * i);
  return r;
}

struct Pair {
  uint64_t x, y;
};

__device__ __forceinline__ Pair weak_seeds(const unsigned char* s, uint64_t a, uint64_t b) {
  const uint64_t w = le64(s), x = le64(s + 8), y = le64(s + 16), z = le64(s + 24);
  a += w;
  b = rotr(b + a + z, 21);
  const uint64_t c = a;
  a += x;
  a += y;
  b += rotr(a, 44);
  return Pair{a + z, b + c};
}

__device__ uint64_t fp64_bytes(const unsigned char* s, uint64_t len) {
  if (len <= 16) {
    if (len >= 8) {
      const uint64_t mul = kC2 + len * 2;
      const uint64_t a = le64(s) + kC2;
      const uint64_t b = le64(s + len - 8);
      return mix16(rotr(b, 37) * mul + a, (rotr(a, 25) + b) * mul, mul);
    }
    if (len >= 4) {
      const uint64_t mul = kC2 + len * 2;
      return mix16(len + (le32(s) << 3), le32(s + len - 4), mul);
    }
    if (len > 0) {
      const uint32_t y = static_cast<uint32_t>(s[0]) + (static_cast<uint32_t>(s[len >> 1]) << 8);
      const uint32_t z = static_cast<uint32_t>(len) + (static_cast<uint32_t>(s[len - 1]) << 2);
      return smix(y * kC2 ^ z * kC0) * kC2;
    }
    return kC2;
  }
  if (len <= 32) {
    const uint64_t mul = kC2 + len * 2;
    const uint64_t a = le64(s) * kC1;
    const uint64_t b = le64(s + 8);
    const uint64_t c = le64(s + len - 8) * mul;
    const uint64_t d = le64(s + len - 16) * kC2;
    return mix16(rotr(a + b, 43) + rotr(c, 30) + d, a + rotr(b + kC2, 18) + c, mul);
  }
  if (len <= 64) {
    const uint64_t mul = kC2 + len * 2;
    const uint64_t a = le64(s) * kC2;
    const uint64_t b = le64(s + 8);
    const uint64_t c = le64(s + len - 8) * mul;
    const uint64_t d = le64(s + len - 16) * kC2;
    const uint64_t y = rotr(a + b, 43) + rotr(c, 30) + d;
    const uint64_t z = mix16(y, a + rotr(b + kC2, 18) + c, mul);
    const uint64_t e = le64(s + 16) * mul;
    const uint64_t f = le64(s + 24);
    const uint64_t g = (y + le64(s + len - 32)) * mul;
    const uint64_t h = (z + le64(s + len - 24)) * mul;
    return mix16(rotr(e + f, 43) + rotr(g, 30) + h, e + rotr(f + a, 18) + g, mul);
  }
  const uint64_t seed = 81;
  uint64_t x = seed;
  uint64_t y = seed * kC1 + 113;
  uint64_t z = smix(y * kC2 + 113) * kC2;
  Pair v{0, 0}, w{0, 0};
  x = x * kC2 + le64(s);
  const unsigned char* end = s + ((len - 1) / 64) * 64;
  const unsigned char* last64 = end + ((len - 1) & 63) - 63;
  do {
    x = rotr(x + y + v.x + le64(s + 8), 37) * kC1;
    y = rotr(y + v.y + le64(s + 48), 42) * kC1;
    x ^= w.y;
    y += v.x + le64(s + 40);
    z = rotr(z + w.x, 33) * kC1;
    v = weak_seeds(s, v.y * kC1, x + w.x);
    w = weak_seeds(s + 32, z + w.y, y + le64(s + 16));
    const uint64_t t = z;
    z = x;
    x = t;
    s += 64;
  } while (s != end);
  const uint64_t mul = kC1 + ((z & 0xff) << 1);
  s = last64;
  w.x += ((len - 1) & 63);
  v.x += w.x;
  w.x += v.x;
  x = rotr(x + y + v.x + le64(s + 8), 37) * mul;
  y = rotr(y + v.y + le64(s + 48), 42) * mul;
  x ^= w.y * 9;
  y += v.x * 9 + le64(s + 40);
  z = rotr(z + w.x, 33) * mul;
  v = weak_seeds(s, v.y * mul, x + w.x);
  w = weak_seeds(s + 32, z + w.y, y + le64(s + 16));
  return mix16(mix16(v.x, w.x, mul) + smix(y) * kC0 + x, mix16(v.y, w.y, mul) + z, mul);
}

// ---------------------------------------------------------------------------
// Fingerprint64 of the decimal text of an int64, built in registers.
// ---------------------------------------------------------------------------
// Two ASCII digits of p < 100, tens in the low byte: p / 10 as (p * 103) >> 10
// (exact below 179) on the full-rate 24-bit multiplier.
__device__ __forceinline__ uint32_t ascii_pair(uint32_t p) {
  const uint32_t t = __umul24(p, 103u) >> 10;
  return 0x3030u + t + ((p - __umul24(t, 10u)) << 8);
}

// x < 10^8 rendered as 8 ASCII digits, first digit in byte 0: one
// multiply-high splits off the upper four digits, the rest are 24-bit
// multiplies (x / 100 as (x * 5243) >> 19, exact below 43699).
__device__ __forceinline__ uint64_t ascii8(uint32_t x) {
  const uint32_t a = x / 10000u;
  const uint32_t b = x - __umul24(a, 10000u);
  const uint32_t a1 = __umul24(a, 5243u) >> 19, b1 = __umul24(b, 5243u) >> 19;
  const uint32_t a2 = a - __umul24(a1, 100u), b2 = b - __umul24(b1, 100u);
  const uint32_t lo = ascii_pair(a1) | (ascii_pair(a2) << 16);
  const uint32_t hi = ascii_pair(b1) | (ascii_pair(b2) << 16);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// x < 1000 rendered as 3 ASCII digits (x / 100 as (x * 41) >> 12, exact
// below 1000).
__device__ __forceinline__ uint64_t ascii3(uint32_t x) {
  const uint32_t h = __umul24(x, 41u) >> 12;
  return (0x30u + h) | (ascii_pair(x - __umul24(h, 100u)) << 8);
}

constexpr uint64_t kAsciiZeros = 0x3030303030303030ull;

// Eight bytes starting at bit s (a multiple of 8, possibly 0) of the 128-bit
// little-endian value hi_w:lo_w.
__device__ __forceinline__ uint64_t window64(uint64_t lo_w, uint64_t hi_w, uint32_t s) {
  return (lo_w >> s) | ((hi_w << 1) << (63u - s));
}

// Leading '0' characters of an 8-digit ASCII group (digit 0 in byte 0); bit
// 63 caps the count at 7 for an all-zero group.
__device__ __forceinline__ uint32_t leading_zero_digits(uint64_t text8) {
  return static_cast<uint32_t>(__builtin_ctzll((text8 ^ kAsciiZeros) | (1ull << 63))) >> 3;
}

// farmhashna::Hash64 of the decimal text of v (TensorFlow's AsString of an
// int64: optional '-', no leading zeros; at most 20 bytes, so only the
// 0-16 and 17-32 byte branches exist).
// The 19 zero-padded digits of |v| sit right-aligned in a 24-byte string P
// held in q0, q1, q2: P[2,5) digits 0-2, P[5,13) digits 3-10, P[13,21)
// digits 11-18.  A text of len bytes is P[21-len, 21), the sign replacing
// the byte before the first digit.  Reads at a fixed distance from the end
// of the text are then fixed registers (the last 8 bytes are digits 11-18,
// the 8 before them digits 3-10); only reads from the start shift by
// 21 - len.
__device__ __forceinline__ uint64_t fp64_decimal(int64_t v) {
  const bool neg = v < 0;
  const uint64_t u = neg ? 0ull - static_cast<uint64_t>(v) : static_cast<uint64_t>(v);
  // u = hi * 10^16 + mid * 10^8 + lo; 10^8 = 390625 * 2^8, so the second
  // division runs on q1 >> 8 < 2^29 in 32 bits
  const uint64_t q1 = u / 100000000ull;
  const uint32_t lo = static_cast<uint32_t>(u) - static_cast<uint32_t>(q1) * 100000000u;
  const uint32_t hi = static_cast<uint32_t>(q1 >> 8) / 390625u;  // <= 922
  const uint32_t mid = static_cast<uint32_t>(q1) - (__umul24(hi, 390625u) << 8);
  const uint64_t d3 = ascii3(hi);
  const uint64_t m8 = ascii8(mid);
  const uint64_t l8 = ascii8(lo);
  const uint32_t nd = hi    ? 17u + (hi >= 10u) + (hi >= 100u)
                      : mid ? 16u - leading_zero_digits(m8)
                            : 8u - leading_zero_digits(l8);
  const uint32_t len = nd + (neg ? 1u : 0u);  // 1..20
  const uint64_t p0 = (d3 << 16) | (m8 << 40);
  const uint64_t p1 = (m8 >> 24) | (l8 << 40);
  const uint64_t p2 = l8 >> 24;
  const uint32_t start = 21u - len;
  const uint64_t mul = kC2 + 2ull * len;
  if (len > 16) {  // HashLen17to32; start = 1..4
    const uint32_t s = 8u * start;
    uint64_t a = (p0 >> s) | (p1 << (64u - s));
    const uint64_t b = (p1 >> s) | (p2 << (64u - s));
    if (neg) a = (a & ~0xffull) | 0x2Dull;
    a *= kC1;
    const uint64_t c = l8 * mul;
    const uint64_t d = m8 * kC2;
    return mix16(rotr(a + b, 43) + rotr(c, 30) + d, a + rotr(b + kC2, 18) + c, mul);
  }
  // first eight bytes of the text (start = 5..20)
  const uint32_t w = start >> 3;
  const uint64_t lo_w = w == 0 ? p0 : (w == 1 ? p1 : p2);
  const uint64_t hi_w = w == 0 ? p1 : (w == 1 ? p2 : 0ull);
  uint64_t a = window64(lo_w, hi_w, 8u * (start & 7u));
  if (neg) a = (a & ~0xffull) | 0x2Dull;
  if (len >= 8) {  // HashLen0to16, 8..16 bytes; the last 8 are digits 11-18
    const uint64_t b = len == 8 ? a : l8;
    const uint64_t a2 = a + kC2;
    return mix16(rotr(b, 37) * mul + a2, (rotr(a2, 25) + b) * mul, mul);
  }
  if (len >= 4) {  // 4..7 bytes; the last 4 are digits 15-18
    const uint64_t x = a & 0xffffffffull;
    const uint64_t y = len == 4 ? x : (l8 >> 32);
    return mix16(len + (x << 3), y, mul);
  }
  const uint32_t c0 = static_cast<uint32_t>(a & 0xff);  // 1..3 bytes
  const uint32_t cm = static_cast<uint32_t>((a >> (8u * (len >> 1))) & 0xff);
  const uint32_t cl = static_cast<uint32_t>((a >> (8u * (len - 1u))) & 0xff);
  const uint32_t y = c0 + (cm << 8);
  const uint32_t z = len + (cl << 2);
  return smix(y * kC2 ^ z * kC0) * kC2;
}

// ---------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t string_len(const unsigned char* p, int64_t span, int nul) {
  if (!nul) return static_cast<uint64_t>(span);
  int64_t i = 0;
  while (i < span && p[i] != 0) ++i;
  return static_cast<uint64_t>(i);
}

__global__ __launch_bounds__(kThreads) void fingerprint_kernel(const char* __restrict__ bytes,
                                                               const int64_t* __restrict__ offsets,
                                                               int64_t n, int nul,
                                                               uint64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const unsigned char* p = reinterpret_cast<const unsigned char*>(bytes) + offsets[i];
  out[i] = fp64_bytes(p, string_len(p, offsets[i + 1] - offsets[i], nul));
}

// bucket of every string; empty strings (span 0) get `empty_value`.
__global__ __launch_bounds__(kThreads) void bucket_strings_kernel(
    const char* __restrict__ bytes, const int64_t* __restrict__ offsets, int64_t n, int nul,
    U64Divisor dv, int64_t empty_value, int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t span = offsets[i + 1] - offsets[i];
  if (span == 0 && empty_value != 0) {
    out[i] = empty_value;
    return;
  }
  const unsigned char* p = reinterpret_cast<const unsigned char*>(bytes) + offsets[i];
  out[i] = static_cast<int64_t>(mod_invariant(fp64_bytes(p, string_len(p, span, nul)), dv));
}

__global__ __launch_bounds__(kThreads) void bucket_int64_kernel(const int64_t* __restrict__ ids,
                                                                int64_t n, U64Divisor dv,
                                                                int64_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  out[i] = static_cast<int64_t>(mod_invariant(fp64_decimal(ids[i]), dv));
}

// out[i,:] = table[bucket[i],:] (exact copy) or zeros when bucket[i] is
// negative or >= rows.
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const float* __restrict__ table,
                                                               int64_t rows, int64_t dim,
                                                               const int64_t* __restrict__ bucket,
                                                               int64_t n, float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= n * dim) return;
  const int64_t i = t / dim, d = t % dim;
  const int64_t b = bucket[i];
  out[t] = (b >= 0 && b < rows) ? table[b * dim + d] : 0.0f;
}

struct FieldSet {
  const float* table[kMaxFields];
  int64_t rows[kMaxFields];
  U64Divisor div[kMaxFields];
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kRawBufferFlags = 0x00020000;  // dword3 of a raw buffer descriptor (gfx950)
// Cache policy of a buffer store (gfx950: bit 1 = nt).  Pooled output rows are
// written once and read only by later kernels, so they go to memory without
// filling L2 and the end-of-kernel release has no dirty lines to write back.
constexpr int kNonTemporal = 2;
constexpr uint32_t kMaskedOff = 0x80000000u;  // past the range check of any table < 2 GiB

// Fused multi-field hash -> bucket -> gather -> pool, one run of consecutive
// bags of one field per wave (G lanes per bag, 64/G bags).  The wave's bags
// occupy a contiguous range of positions, so lane l loads and hashes
// position wbeg + 64k + l -- every lane hashes one id per 64 positions, the
// id loads are coalesced -- and turns the bucket into the byte offset of its
// row.  Each bag group then walks its positions eight at a time, fetching
// the offset from the lane that hashed it (ds_bpermute) and the row chunk
// through a raw buffer load; positions past the bag carry an offset past
// the buffer's range check and read zeros, which leave the +0-seeded,
// index-ordered sums unchanged.
template <int G, bool MEAN>
__global__ __launch_bounds__(kThreads) void hashed_bags_wave_kernel(
    FieldSet fs, int64_t field0, int64_t nfields, int64_t batch, int64_t dim,
    int64_t waves_per_field, const int64_t* __restrict__ ids, const int64_t* __restrict__ offsets,
    float* __restrict__ out, int64_t ldo, int64_t* __restrict__ buckets_out) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int NB = 64 / G;
  const int lane = threadIdx.x & 63;
  const int64_t w =
      (int64_t)blockIdx.x * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w >= nfields * waves_per_field) return;
  const int fl = static_cast<int>(w / waves_per_field);
  const int64_t b0 = (w - (int64_t)fl * waves_per_field) * NB;
  const int64_t f = field0 + fl;
  const int64_t nbag = batch - b0 < NB ? batch - b0 : NB;  // bags of this wave
  const int64_t wbeg = offsets[f * batch + b0];
  const int64_t wend = offsets[f * batch + b0 + nbag];
  const int grp = lane / G;
  const int g = lane & (G - 1);
  const bool bag_ok = grp < nbag;
  const int64_t b = b0 + (bag_ok ? grp : 0);
  const int64_t beg = bag_ok ? offsets[f * batch + b] : wend;
  const int64_t end = bag_ok ? offsets[f * batch + b + 1] : wend;
  const U64Divisor dv = fs.div[fl];
  const uint32_t row_bytes = static_cast<uint32_t>(dim * sizeof(float));
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(fs.table[fl]), 0, static_cast<int>(fs.rows[fl] * row_bytes),
      kRawBufferFlags);
  float* __restrict__ dst = out + b * ldo + f * dim;
  for (int64_t c0 = 0; c0 < dim; c0 += (int64_t)G * 4) {
    const int64_t c = c0 + (int64_t)g * 4;
    const bool active = c < dim;
    const uint32_t c_off = active ? static_cast<uint32_t>(c * sizeof(float)) : kMaskedOff;
    f32x4 acc = f32x4(0.0f);
    for (int64_t k0 = wbeg; k0 < wend; k0 += 64) {
      const int64_t p = k0 + lane;
      const bool pv = p < wend;
      const int64_t id = ids[pv ? p : wend - 1];
      const uint64_t bucket = mod_invariant(fp64_decimal(id), dv);
      if (buckets_out && pv && c0 == 0) buckets_out[p] = static_cast<int64_t>(bucket);
      const uint32_t my_off = pv ? static_cast<uint32_t>(bucket) * row_bytes : kMaskedOff;
      // this bag's positions inside the chunk: [lo, lo + cnt) relative to k0
      const int64_t lo64 = beg > k0 ? beg : k0;
      const int64_t hi64 = end < k0 + 64 ? end : k0 + 64;
      const int cnt = hi64 > lo64 ? static_cast<int>(hi64 - lo64) : 0;
      const int lo = static_cast<int>(lo64 - k0);
      for (int u0 = 0; __ballot(cnt > u0) != 0; u0 += 8) {
        f32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int u = u0 + i;
          const uint32_t off = static_cast<uint32_t>(
              __builtin_amdgcn_ds_bpermute(((lo + u) & 63) << 2, static_cast<int>(my_off)));
          const u32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(
              rsrc, static_cast<int>((u < cnt ? off : kMaskedOff) + c_off), 0, 0);
          v[i] = __builtin_bit_cast(f32x4, raw);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += v[i];
      }
    }
    if (MEAN) {
      const int32_t n = static_cast<int32_t>(end - beg);
      if (n > 0) acc *= 1.0f / static_cast<float>(n);
    }
    if (active && bag_ok) __builtin_nontemporal_store(acc, reinterpret_cast<f32x4*>(dst + c));
  }
}

template <int G>
void launch_hashed_wave_g(const FieldSet& fs, int64_t f0, int64_t nf, int64_t batch, int64_t dim,
                          const int64_t* ids, const int64_t* offsets, int combiner, float* out,
                          int64_t ldo, int64_t* buckets_out, hipStream_t s) {
  const int64_t wpf = (batch + 64 / G - 1) / (64 / G);
  dim3 grid((unsigned)ceil_div(nf * wpf, kThreads / 64));
  if (combiner == ANNC_COMBINER_MEAN)
    hipLaunchKernelGGL((hashed_bags_wave_kernel<G, true>), grid, dim3(kThreads), 0, s, fs, f0, nf,
                       batch, dim, wpf, ids, offsets, out, ldo, buckets_out);
  else
    hipLaunchKernelGGL((hashed_bags_wave_kernel<G, false>), grid, dim3(kThreads), 0, s, fs, f0,
                       nf, batch, dim, wpf, ids, offsets, out, ldo, buckets_out);
}

// ---------------------------------------------------------------------------
// Pipelined hashed bags for rows of at most 16 floats.
// ---------------------------------------------------------------------------
// A run is 16 consecutive bags of one field; bag j of a run belongs to the
// lane group j (4 lanes, 4 floats each).  A wave walks a contiguous range of
// runs (field-major) with a three-deep software pipeline, so that the row
// gathers of one run are in flight while the next run is hashed:
//   offsets of run i+3 and ids of run i+2 are loaded,
//   run i+1 is hashed and its row loads are issued,
//   run i's rows (issued one step earlier) are summed and stored.
// A run whose positions span more than two 64-position chunks takes the
// synchronous path of hashed_bags_wave_kernel instead.
constexpr int kPipeBags = 16;  // bags per run
constexpr int kPipeU = 8;      // positions per bag whose rows are issued in one batch

struct RunCursor {  // run = (field fl of the launch, run j within the field)
  int64_t fl, j;
};

__device__ __forceinline__ void advance(RunCursor& c, int64_t runs_per_field) {
  if (++c.j == runs_per_field) {
    c.j = 0;
    ++c.fl;
  }
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32), l);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int64_t shfl64(int64_t v, int src_lane) {
  const int lo = __builtin_amdgcn_ds_bpermute(src_lane << 2, static_cast<int>(v));
  const int hi = __builtin_amdgcn_ds_bpermute(src_lane << 2, static_cast<int>(v >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                              static_cast<uint32_t>(lo));
}

// Row chunk of position q (relative to the run's first position) from the
// lane that hashed it.
__device__ __forceinline__ uint32_t row_offset_of(int q, uint32_t off0, uint32_t off1,
                                                  bool two_chunks) {
  const uint32_t a = static_cast<uint32_t>(
      __builtin_amdgcn_ds_bpermute((q & 63) << 2, static_cast<int>(off0)));
  if (!two_chunks) return a;
  const uint32_t b = static_cast<uint32_t>(
      __builtin_amdgcn_ds_bpermute((q & 63) << 2, static_cast<int>(off1)));
  return q < 64 ? a : b;
}

// Five waves a SIMD: the kernel needs 97 VGPRs unconstrained (four waves);
// at 96 it keeps every value in registers (a few scalars move to VGPR
// lanes) and configs[3] runs 16.75 against 16.91 us.
template <bool MEAN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(5))) void hashed_bags_pipe_kernel(
    FieldSet fs, int64_t field0, int64_t batch, int64_t dim, int64_t runs_per_field,
    int64_t total_runs, int64_t runs_per_wave, const int64_t* __restrict__ ids,
    const int64_t* __restrict__ offsets, float* __restrict__ out, int64_t ldo,
    int64_t* __restrict__ buckets_out) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  // Prefetched offsets (two runs) and ids (one run) wait here: a register
  // still waiting on a load must not be carried across the loop's back edge
  // (the copy would wait for every older load, row gathers included).
  // (volatile: the compiler must not forward these stores to the next
  // iteration's loads through registers)
  __shared__ int64_t sh_starts_mem[kThreads / 64][2][64];
  __shared__ int64_t sh_ids_mem[kThreads / 64][2][64];
  typedef volatile __attribute__((address_space(3))) int64_t lds_i64;
  lds_i64(*sh_starts)[2][64] = (lds_i64(*)[2][64])sh_starts_mem;
  lds_i64(*sh_ids)[2][64] = (lds_i64(*)[2][64])sh_ids_mem;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // XCD-aware block order: consecutive hardware blocks go to different XCDs
  // (round robin over 8), so give each XCD a contiguous share of the runs
  // and the L2 of that XCD a few fields' tables.
  const uint32_t nblk = gridDim.x, xcd = blockIdx.x & 7u, k = blockIdx.x >> 3;
  const uint32_t per = nblk >> 3, rem = nblk & 7u;
  const uint32_t blk = xcd * per + (xcd < rem ? xcd : rem) + k;
  const int64_t w = (int64_t)blk * (kThreads / 64) + wid;
  const int64_t r0 = w * runs_per_wave;
  if (r0 >= total_runs) return;
  const int64_t n = total_runs - r0 < runs_per_wave ? total_runs - r0 : runs_per_wave;
  const int grp = lane >> 2;
  const int c = (lane & 3) * 4;
  const bool active = c < dim;
  const uint32_t c_off = active ? static_cast<uint32_t>(c * sizeof(float)) : kMaskedOff;
  const uint32_t row_bytes = static_cast<uint32_t>(dim * sizeof(float));

  auto nbag_of = [&](const RunCursor& rc) -> int {
    const int64_t left = batch - rc.j * kPipeBags;
    return static_cast<int>(left < kPipeBags ? left : kPipeBags);
  };
  // lane l: start of bag min(l, nbag) of the run (the run's end for l >= nbag)
  auto load_starts = [&](const RunCursor& rc) -> int64_t {
    const int nb = nbag_of(rc);
    const int64_t base = (field0 + rc.fl) * batch + rc.j * kPipeBags;
    return offsets[base + (lane < nb ? lane : nb)];
  };
  struct Ids {
    int64_t a, b;  // positions wbeg + lane and wbeg + 64 + lane
  };
  // Always two loads; lanes without a position read offsets[0] instead.
  auto load_ids = [&](const RunCursor& rc, int64_t starts) -> Ids {
    const int nb = nbag_of(rc);
    const int64_t wbeg = readlane64(starts, 0), wend = readlane64(starts, nb);
    const bool ok = wend > wbeg && wend - wbeg <= 128;
    const int64_t p = wbeg + lane;
    const int64_t* pa = ok ? ids + (p < wend ? p : wend - 1) : offsets;
    const int64_t* pb = ok && wend - wbeg > 64 ? ids + (p + 64 < wend ? p + 64 : wend - 1) : offsets;
    return Ids{*pa, *pb};
  };
  auto field_of = [&](const RunCursor& rc) {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(rc.fl));
  };
  auto rsrc_of = [&](const RunCursor& rc) {
    const int fl = field_of(rc);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(fs.table[fl]), 0,
                                             static_cast<int>(fs.rows[fl] * row_bytes),
                                             kRawBufferFlags);
  };
  // The run's 16 output rows through a buffer store: lanes without a bag
  // (or past dim) store past the range and are dropped, so the store is one
  // unconditional instruction.
  auto store = [&](const RunCursor& rc, int cnt, f32x4 acc) {
    if (MEAN && cnt > 0) acc *= 1.0f / static_cast<float>(cnt);
    const int nb = nbag_of(rc);
    float* base = out + (rc.j * kPipeBags) * ldo + (field0 + rc.fl) * dim;
    const auto orsrc = __builtin_amdgcn_make_buffer_rsrc(
        base, 0, static_cast<int>(nb * ldo * static_cast<int64_t>(sizeof(float))), kRawBufferFlags);
    const uint32_t o = active && grp < nb ? static_cast<uint32_t>((grp * ldo + c) * sizeof(float))
                                          : kMaskedOff;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), orsrc,
                                           static_cast<int>(o), 0, kNonTemporal);
  };

  // A hashed run: row byte offsets of its positions, held by the lanes that
  // hashed them (chunk 0: positions wbeg + lane, chunk 1: wbeg + 64 + lane).
  struct Hashed {
    RunCursor rc;
    int64_t starts;
    bool slow, two;
    int rel, cnt;  // this lane group's bag: first position - wbeg, length
    uint32_t off0, off1;
  };
  auto hash_run = [&](const RunCursor& rc, int64_t starts, const Ids& iv) -> Hashed {
    const int nb = nbag_of(rc);
    const int64_t wbeg = readlane64(starts, 0), wend = readlane64(starts, nb);
    Hashed h;
    h.rc = rc;
    h.starts = starts;
    h.slow = wend - wbeg > 128;
    h.two = wend - wbeg > 64;
    h.off0 = kMaskedOff;
    h.off1 = kMaskedOff;
    const int64_t beg = shfl64(starts, grp), end = shfl64(starts, grp + 1);
    h.rel = static_cast<int>(beg - wbeg);
    h.cnt = grp < nb ? static_cast<int>(end - beg) : 0;
    if (h.slow || wend == wbeg) return h;
    const U64Divisor dv = fs.div[field_of(rc)];
    const int64_t p = wbeg + lane;
    const uint64_t b0 = mod_invariant(fp64_decimal(iv.a), dv);
    if (p < wend) {
      h.off0 = static_cast<uint32_t>(b0) * row_bytes;
      if (buckets_out) buckets_out[p] = static_cast<int64_t>(b0);
    }
    if (h.two) {
      const uint64_t b1 = mod_invariant(fp64_decimal(iv.b), dv);
      if (p + 64 < wend) {
        h.off1 = static_cast<uint32_t>(b1) * row_bytes;
        if (buckets_out) buckets_out[p + 64] = static_cast<int64_t>(b1);
      }
    }
    return h;
  };
  // Row loads of positions u0 .. u0+kPipeU-1 of this lane group's bag
  // (masked for a run on the synchronous path).
  auto issue = [&](const Hashed& h, int u0, f32x4* v) {
    const auto rsrc = rsrc_of(h.rc);
    const int cnt = h.slow ? 0 : h.cnt;
    if (h.two) {
#pragma unroll
      for (int i = 0; i < kPipeU; ++i) {
        const int u = u0 + i;
        const uint32_t o = row_offset_of(h.rel + u, h.off0, h.off1, true);
        v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rsrc, static_cast<int>((u < cnt ? o : kMaskedOff) + c_off), 0, 0));
      }
    } else {
#pragma unroll
      for (int i = 0; i < kPipeU; ++i) {
        const int u = u0 + i;
        const uint32_t o = row_offset_of(h.rel + u, h.off0, h.off1, false);
        v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rsrc, static_cast<int>((u < cnt ? o : kMaskedOff) + c_off), 0, 0));
      }
    }
  };
  // Synchronous path for a run of more than 128 positions: 64 at a time,
  // sums carried across chunks in position order.
  auto run_slow = [&](const Hashed& h) {
    const RunCursor& rc = h.rc;
    const int nb = nbag_of(rc);
    const int64_t wbeg = readlane64(h.starts, 0), wend = readlane64(h.starts, nb);
    const int64_t beg = wbeg + h.rel, end = beg + h.cnt;
    const U64Divisor dv = fs.div[field_of(rc)];
    const auto rsrc = rsrc_of(rc);
    f32x4 acc = f32x4(0.0f);
    for (int64_t k0 = wbeg; k0 < wend; k0 += 64) {
      const int64_t p = k0 + lane;
      const bool pv = p < wend;
      const uint64_t bucket = mod_invariant(fp64_decimal(ids[pv ? p : wend - 1]), dv);
      if (buckets_out && pv) buckets_out[p] = static_cast<int64_t>(bucket);
      const uint32_t my_off = pv ? static_cast<uint32_t>(bucket) * row_bytes : kMaskedOff;
      const int64_t lo64 = beg > k0 ? beg : k0;
      const int64_t hi64 = end < k0 + 64 ? end : k0 + 64;
      const int cnt = hi64 > lo64 ? static_cast<int>(hi64 - lo64) : 0;
      const int lo = static_cast<int>(lo64 - k0);
      for (int u0 = 0; __ballot(cnt > u0) != 0; u0 += kPipeU) {
        f32x4 v[kPipeU];
#pragma unroll
        for (int i = 0; i < kPipeU; ++i) {
          const int u = u0 + i;
          const uint32_t o = static_cast<uint32_t>(
              __builtin_amdgcn_ds_bpermute(((lo + u) & 63) << 2, static_cast<int>(my_off)));
          v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rsrc, static_cast<int>((u < cnt ? o : kMaskedOff) + c_off), 0, 0));
        }
#pragma unroll
        for (int i = 0; i < kPipeU; ++i) acc += v[i];
      }
    }
    store(rc, h.cnt, acc);
  };
  // Sum the issued rows (plus further batches for bags longer than kPipeU)
  // and store the run; a run of more than 128 positions is done here.
  auto finish = [&](const Hashed& h, const f32x4* v) {
    if (h.slow) {
      run_slow(h);
      return;
    }
    f32x4 acc = f32x4(0.0f);
#pragma unroll
    for (int i = 0; i < kPipeU; ++i) acc += v[i];
    for (int u0 = kPipeU; __ballot(h.cnt > u0) != 0; u0 += kPipeU) {
      f32x4 w2[kPipeU];
      issue(h, u0, w2);
#pragma unroll
      for (int i = 0; i < kPipeU; ++i) acc += w2[i];
    }
    store(h.rc, h.cnt, acc);
  };

  // Cursors over the wave's runs; the prefetch cursors stop at the last run
  // (its loads are repeated, never used), so every step issues the same
  // loads and each consumer waits only for its own.
  const int64_t last = n - 1;
  RunCursor cs{r0 / runs_per_field, r0 % runs_per_field};  // next offsets load
  RunCursor ci = cs, ch = cs;                              // next ids load, next hash
  int64_t ks = 0, ki = 0;
  auto next = [&](RunCursor& cur, int64_t& kk) {
    if (kk < last) {
      advance(cur, runs_per_field);
      ++kk;
    }
  };
  const int64_t s0 = load_starts(cs);
  next(cs, ks);
  const int64_t s1 = load_starts(cs);
  next(cs, ks);
  const int64_t s2 = load_starts(cs);
  next(cs, ks);
  const Ids i0 = load_ids(ci, s0);
  next(ci, ki);
  const Ids i1 = load_ids(ci, s1);
  next(ci, ki);
  Hashed hc = hash_run(ch, s0, i0);
  advance(ch, runs_per_field);
  sh_starts[wid][1][lane] = s1;
  sh_starts[wid][0][lane] = s2;
  sh_ids[wid][0][lane] = i1.a;
  sh_ids[wid][1][lane] = i1.b;
  // Iteration i issues run i's row loads, hashes run i+1 while they are in
  // flight, then sums and stores run i.  Every load is consumed in the
  // iteration that issued it; only hashed offsets (registers, no pending
  // loads) and LDS carry over.  LDS holds the offsets of runs i+1 and i+2
  // (slots (i+1)&1 and i&1) and the ids of run i+1.
  for (int64_t i = 0; i < n; ++i) {
    f32x4 v[kPipeU];
    issue(hc, 0, v);
    const int64_t spre = sh_starts[wid][i & 1][lane];  // run i+2
    const Ids ipf = load_ids(ci, spre);                // ids of run i+2
    next(ci, ki);
    const int64_t sld = load_starts(cs);               // offsets of run i+3
    next(cs, ks);
    Hashed hn;
    if (i + 1 < n) {
      const Ids inx{sh_ids[wid][0][lane], sh_ids[wid][1][lane]};
      hn = hash_run(ch, sh_starts[wid][(i + 1) & 1][lane], inx);
      advance(ch, runs_per_field);
    }
    finish(hc, v);
    sh_ids[wid][0][lane] = ipf.a;
    sh_ids[wid][1][lane] = ipf.b;
    sh_starts[wid][(i + 1) & 1][lane] = sld;
    hc = hn;
  }
}

template <bool MEAN>
void launch_hashed_pipe(const FieldSet& fs, int64_t f0, int64_t nf, int64_t batch, int64_t dim,
                        const int64_t* ids, const int64_t* offsets, float* out, int64_t ldo,
                        int64_t* buckets_out, int64_t runs_per_wave, hipStream_t s) {
  const int64_t rpf = (batch + kPipeBags - 1) / kPipeBags;
  const int64_t total = nf * rpf;
  const int64_t waves = (total + runs_per_wave - 1) / runs_per_wave;
  dim3 grid((unsigned)ceil_div(waves, kThreads / 64));
  hipLaunchKernelGGL((hashed_bags_pipe_kernel<MEAN>), grid, dim3(kThreads), 0, s, fs, f0, batch,
                     dim, rpf, total, runs_per_wave, ids, offsets, out, ldo, buckets_out);
}

// Fused multi-field hash -> bucket -> gather -> pool with the row offsets
// staged in LDS.  A wave owns a run of BW = (64/G)*R consecutive bags of one
// field.  Phase 1 hashes the run's positions 64 at a time -- every lane busy
// except in the last chunk -- into the wave's LDS window as row byte offsets
// (positions past the run carry an offset past the buffer's range check).
// Phase 2: the 64/G lane groups take R bags each (bag r*(64/G) + group), G
// lanes per bag with 4 floats per lane, and walk the bags in index order,
// reading offsets from LDS and rows through raw buffer loads, all R bags'
// loads in flight together.  A run longer than the window is processed in
// windows, the sums carried across them in position order.  Requires
// dim <= 4G (one column pass).
template <int G, int R, bool MEAN>
__global__ __launch_bounds__(kThreads) void hashed_bags_lds_kernel(
    FieldSet fs, int64_t field0, int64_t nfields, int64_t batch, int64_t dim,
    int64_t waves_per_field, const int64_t* __restrict__ ids, const int64_t* __restrict__ offsets,
    float* __restrict__ out, int64_t ldo, int64_t* __restrict__ buckets_out) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int NB = 64 / G;   // lane groups
  constexpr int BW = NB * R;   // bags per wave
  static_assert(BW <= 64, "one bag start per lane");
  constexpr int kChunks = 4;   // 64-position chunks per window
  constexpr int kWin = 64 * kChunks;
  constexpr int U = 4;         // positions per bag per round
  __shared__ uint32_t win_off[kThreads / 64][kWin];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t w = (int64_t)blockIdx.x * (kThreads / 64) + wid;
  if (w >= nfields * waves_per_field) return;
  const int fl = static_cast<int>(w / waves_per_field);
  const int64_t b0 = (w - (int64_t)fl * waves_per_field) * BW;
  const int64_t f = field0 + fl;
  const int nbag = static_cast<int>(batch - b0 < BW ? batch - b0 : BW);
  const int64_t* __restrict__ run = offsets + f * batch + b0;
  const int64_t wbeg = run[0];
  const int64_t wend = run[nbag];
  // lane i < nbag holds the start of bag i; the others hold the run's end
  const int64_t start = run[lane < nbag ? lane : nbag];
  const int grp = lane / G;
  const int g = lane & (G - 1);
  int64_t beg[R], end[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int j = r * NB + grp;
    beg[r] = __shfl(start, j, 64);
    const int64_t nx = __shfl(start, (j + 1) & 63, 64);
    end[r] = j + 1 < 64 ? nx : wend;
  }
  const U64Divisor dv = fs.div[fl];
  const uint32_t row_bytes = static_cast<uint32_t>(dim * sizeof(float));
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(fs.table[fl]), 0, static_cast<int>(fs.rows[fl] * row_bytes),
      kRawBufferFlags);
  const int c = g * 4;
  const bool active = c < dim;
  const uint32_t c_off = active ? static_cast<uint32_t>(c * sizeof(float)) : kMaskedOff;
  uint32_t* __restrict__ win = win_off[wid];
  f32x4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f32x4(0.0f);

  for (int64_t w0 = wbeg; w0 < wend; w0 += kWin) {
    const int64_t wlen64 = wend - w0 < kWin ? wend - w0 : kWin;
    const int wlen = static_cast<int>(wlen64);
    // ids of the window, all loads issued before any hashing
    int64_t idv[kChunks];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      const int q = 64 * ch + lane;
      idv[ch] = ids[w0 + (q < wlen ? q : wlen - 1)];
    }
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
      if (64 * ch < wlen) {
        const int q = 64 * ch + lane;
        const uint64_t bucket = mod_invariant(fp64_decimal(idv[ch]), dv);
        win[q] = q < wlen ? static_cast<uint32_t>(bucket) * row_bytes : kMaskedOff;
        if (buckets_out && q < wlen) buckets_out[w0 + q] = static_cast<int64_t>(bucket);
      }
    }
    // LDS writes of this wave are visible to its own later reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int lo[R], cnt[R];
    bool more = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t l = beg[r] > w0 ? beg[r] : w0;
      const int64_t h = end[r] < w0 + wlen ? end[r] : w0 + wlen;
      lo[r] = static_cast<int>(l - w0);
      cnt[r] = h > l ? static_cast<int>(h - l) : 0;
      more = more || cnt[r] > 0;
    }
    for (int u0 = 0; __ballot(more) != 0; u0 += U) {
      f32x4 v[R][U];
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < U; ++i) {
          const int u = u0 + i;
          const uint32_t off = win[(lo[r] + u) & (kWin - 1)];
          const u32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(
              rsrc, static_cast<int>((u < cnt[r] ? off : kMaskedOff) + c_off), 0, 0);
          v[r][i] = __builtin_bit_cast(f32x4, raw);
        }
      more = false;
#pragma unroll
      for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int i = 0; i < U; ++i) acc[r] += v[r][i];
        more = more || cnt[r] > u0 + U;
      }
    }
    // the next window's LDS writes must not pass this window's reads
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int j = r * NB + grp;
    if (MEAN) {
      const int32_t n = static_cast<int32_t>(end[r] - beg[r]);
      if (n > 0) acc[r] *= 1.0f / static_cast<float>(n);
    }
    if (active && j < nbag)
      __builtin_nontemporal_store(acc[r],
                                  reinterpret_cast<f32x4*>(out + (b0 + j) * ldo + f * dim + c));
  }
}

template <int G, int R>
void launch_hashed_lds_g(const FieldSet& fs, int64_t f0, int64_t nf, int64_t batch, int64_t dim,
                         const int64_t* ids, const int64_t* offsets, int combiner, float* out,
                         int64_t ldo, int64_t* buckets_out, hipStream_t s) {
  constexpr int BW = (64 / G) * R;
  const int64_t wpf = (batch + BW - 1) / BW;
  dim3 grid((unsigned)ceil_div(nf * wpf, kThreads / 64));
  if (combiner == ANNC_COMBINER_MEAN)
    hipLaunchKernelGGL((hashed_bags_lds_kernel<G, R, true>), grid, dim3(kThreads), 0, s, fs, f0,
                       nf, batch, dim, wpf, ids, offsets, out, ldo, buckets_out);
  else
    hipLaunchKernelGGL((hashed_bags_lds_kernel<G, R, false>), grid, dim3(kThreads), 0, s, fs, f0,
                       nf, batch, dim, wpf, ids, offsets, out, ldo, buckets_out);
}

// Fused multi-field hash -> bucket -> gather -> pool.  A bag is owned by a
// group of G lanes (4 floats of the row each).  The group hashes up to G
// ids at once (one per lane), then every lane walks the bag in index order,
// taking each bucket from the lane that hashed it.
template <int G, bool MEAN>
__global__ __launch_bounds__(kThreads) void hashed_bags_kernel(
    FieldSet fs, int64_t field0, int64_t nfields, int64_t batch, int64_t dim,
    const int64_t* __restrict__ ids, const int64_t* __restrict__ offsets,
    float* __restrict__ out, int64_t ldo, int64_t* __restrict__ buckets_out) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int g = threadIdx.x & (G - 1);
  const int64_t local = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / G;
  if (local >= nfields * batch) return;
  const int64_t fl = local / batch;  // field within this launch
  const int64_t b = local - fl * batch;
  const int64_t bag = (field0 + fl) * batch + b;
  const int64_t beg = offsets[bag];
  const int64_t end = offsets[bag + 1];
  const float* __restrict__ table = fs.table[fl];
  const U64Divisor dv = fs.div[fl];
  float* __restrict__ dst = out + b * ldo + (field0 + fl) * dim;
  // Every lane of the group runs the same chunk and id loops (the shuffles
  // read buckets from all G lanes); lanes past `dim` only skip the row math.
  for (int64_t base = 0; base < dim; base += (int64_t)G * 4) {
    const int64_t c = base + (int64_t)g * 4;
    const bool active = c < dim;
    f32x4 acc = f32x4(0.0f);
    for (int64_t j0 = beg; j0 < end; j0 += G) {
      int64_t mine = 0;
      if (j0 + g < end) {
        mine = static_cast<int64_t>(mod_invariant(fp64_decimal(ids[j0 + g]), dv));
        if (buckets_out && base == 0) buckets_out[j0 + g] = mine;
      }
      const int cnt = (int)((end - j0) < G ? (end - j0) : G);
      for (int u = 0; u < cnt; ++u) {
        const int64_t r = __shfl(mine, u, G);
        if (active) acc += *reinterpret_cast<const f32x4*>(table + r * dim + c);
      }
    }
    if (MEAN) {
      const int32_t cnt = static_cast<int32_t>(end - beg);
      if (cnt > 0) acc *= 1.0f / static_cast<float>(cnt);
    }
    if (active) *reinterpret_cast<f32x4*>(dst + c) = acc;
  }
}

template <int G>
void launch_hashed_g(const FieldSet& fs, int64_t f0, int64_t nf, int64_t batch, int64_t dim,
                     const int64_t* ids, const int64_t* offsets, int combiner, float* out,
                     int64_t ldo, int64_t* buckets_out, hipStream_t s) {
  dim3 grid((unsigned)ceil_div(nf * batch * G, kThreads));
  if (combiner == ANNC_COMBINER_MEAN)
    hipLaunchKernelGGL((hashed_bags_kernel<G, true>), grid, dim3(kThreads), 0, s, fs, f0, nf,
                       batch, dim, ids, offsets, out, ldo, buckets_out);
  else
    hipLaunchKernelGGL((hashed_bags_kernel<G, false>), grid, dim3(kThreads), 0, s, fs, f0, nf,
                       batch, dim, ids, offsets, out, ldo, buckets_out);
}

// KPFusedSparseEmbedding support: keep[i] = empty || bucket > 0.
__global__ void sparse_embedding_flags_kernel(const int64_t* __restrict__ offsets,
                                              const int64_t* __restrict__ bucket, int64_t n,
                                              int32_t* __restrict__ keep) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const bool empty = offsets[i + 1] == offsets[i];
  keep[i] = (empty || bucket[i] > 0) ? 1 : 0;
}

__global__ void sparse_embedding_scatter_kernel(const int64_t* __restrict__ offsets,
                                                const int64_t* __restrict__ bucket,
                                                const int32_t* __restrict__ keep,
                                                const int32_t* __restrict__ pos, int64_t n,
                                                int64_t* __restrict__ indices,
                                                int64_t* __restrict__ values,
                                                uint8_t* __restrict__ empty) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  indices[2 * i] = i;
  indices[2 * i + 1] = 0;
  if (keep[i]) {
    const bool e = offsets[i + 1] == offsets[i];
    values[pos[i]] = e ? 0 : bucket[i];
    empty[pos[i]] = e ? 1 : 0;
  }
}

}  // namespace

// Internal launchers used by the TF-op entry points (tf_ops.cpp).
int launch_bucket_strings(hipStream_t s, const char* bytes, const int64_t* offsets, int64_t n,
                          int64_t num_buckets, int nul, int64_t empty_value, int64_t* out) {
  if (n == 0) return ANNC_OK;
  hipLaunchKernelGGL(bucket_strings_kernel, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads),
                     0, s, bytes, offsets, n, nul, make_divisor((uint64_t)num_buckets),
                     empty_value, out);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

int launch_gather_rows(hipStream_t s, const float* table, int64_t rows, int64_t dim,
                       const int64_t* bucket, int64_t n, float* out) {
  if (n * dim == 0) return ANNC_OK;
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)ceil_div(n * dim, kThreads)),
                     dim3(kThreads), 0, s, table, rows, dim, bucket, n, out);
  ANNC_HIP_TRY(hipGetLastError());
  return ANNC_OK;
}

int run_sparse_embedding(hipStream_t s, const int64_t* offsets, const int64_t* bucket, int64_t n,
                         int32_t* keep, int32_t* pos, int64_t* indices, int64_t* values,
                         uint8_t* empty, int64_t* num_values) {
  if (n == 0) {
    *num_values = 0;
    return ANNC_OK;
  }
  const dim3 grid((unsigned)ceil_div(n, kThreads));
  hipLaunchKernelGGL(sparse_embedding_flags_kernel, grid, dim3(kThreads), 0, s, offsets, bucket, n,
                     keep);
  ANNC_HIP_TRY(hipGetLastError());
  void* temp = stream_workspace(s, scan_temp_bytes(n));
  if (!temp) return set_error(ANNC_RESOURCE_EXHAUSTED, "workspace allocation failed");
  int rc = exclusive_sum(s, keep, pos, n, temp);
  if (rc != ANNC_OK) return rc;
  hipLaunchKernelGGL(sparse_embedding_scatter_kernel, grid, dim3(kThreads), 0, s, offsets, bucket,
                     keep, pos, n, indices, values, empty);
  ANNC_HIP_TRY(hipGetLastError());
  int32_t last[2];
  rc = read_back(s, {{&last[0], pos + n - 1, sizeof(int32_t)},
                               {&last[1], keep + n - 1, sizeof(int32_t)}});
  if (rc != ANNC_OK) return rc;
  *num_values = (int64_t)last[0] + last[1];
  return ANNC_OK;
}

}  // namespace annc

extern "C" {

int annc_hip_fingerprint64(void* stream, const char* bytes, const int64_t* offsets, int64_t n,
                           int nul_terminated, uint64_t* out) {
  using namespace annc;
  ANNC_REQUIRE(n >= 0, "negative count");
  if (n == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(bytes && offsets && out, "null pointer");
  hipLaunchKernelGGL(fingerprint_kernel, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), bytes, offsets, n, nul_terminated, out);
  ANNC_HIP_TRY(hipGetLastError());
  return set_error(ANNC_OK, "");
}

int annc_hip_hash_bucket_strings(void* stream, const char* bytes, const int64_t* offsets,
                                 int64_t n, int64_t num_buckets, int nul_terminated,
                                 int64_t* buckets) {
  using namespace annc;
  ANNC_REQUIRE(n >= 0, "negative count");
  ANNC_REQUIRE(num_buckets >= 1, "num_buckets must be >= 1");
  if (n == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(bytes && offsets && buckets, "null pointer");
  int rc = launch_bucket_strings(static_cast<hipStream_t>(stream), bytes, offsets, n, num_buckets,
                                 nul_terminated, 0, buckets);
  return rc == ANNC_OK ? set_error(ANNC_OK, "") : rc;
}

int annc_hip_hash_bucket_int64(void* stream, const int64_t* ids, int64_t n, int64_t num_buckets,
                               int64_t* buckets) {
  using namespace annc;
  ANNC_REQUIRE(n >= 0, "negative count");
  ANNC_REQUIRE(num_buckets >= 1, "num_buckets must be >= 1");
  if (n == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(ids && buckets, "null pointer");
  hipLaunchKernelGGL(bucket_int64_kernel, dim3((unsigned)ceil_div(n, kThreads)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), ids, n,
                     make_divisor(static_cast<uint64_t>(num_buckets)), buckets);
  ANNC_HIP_TRY(hipGetLastError());
  return set_error(ANNC_OK, "");
}

int annc_hip_hashed_embedding_bags(void* stream, int64_t num_fields, int64_t batch, int64_t dim,
                                   const float* const* tables, const int64_t* table_rows,
                                   const int64_t* num_buckets, const int64_t* ids,
                                   const int64_t* offsets, int combiner, float* out, int64_t ldo,
                                   int64_t* buckets_out) {
  using namespace annc;
  ANNC_REQUIRE(num_fields >= 0 && batch >= 0 && dim >= 1, "bad dimensions");
  ANNC_REQUIRE(combiner == ANNC_COMBINER_SUM || combiner == ANNC_COMBINER_MEAN,
               "combiner must be 0 or 1");
  ANNC_REQUIRE(ldo >= num_fields * dim, "ldo < num_fields * dim");
  if (num_fields == 0 || batch == 0) return set_error(ANNC_OK, "");
  ANNC_REQUIRE(tables && table_rows && num_buckets && ids && offsets && out, "null pointer");
  ANNC_REQUIRE(dim % 4 == 0 && ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "hashed bags need dim and ldo multiples of 4 and a 16-byte aligned output");
  for (int64_t f = 0; f < num_fields; ++f) {
    ANNC_REQUIRE(num_buckets[f] >= 1, "num_buckets must be >= 1 (field %lld)", (long long)f);
    ANNC_REQUIRE(num_buckets[f] <= table_rows[f],
                 "num_buckets %lld exceeds the %lld table rows of field %lld",
                 (long long)num_buckets[f], (long long)table_rows[f], (long long)f);
    ANNC_REQUIRE(tables[f] && (reinterpret_cast<uintptr_t>(tables[f]) & 15) == 0,
                 "table of field %lld is null or not 16-byte aligned", (long long)f);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t lanes = dim / 4;
  for (int64_t f0 = 0; f0 < num_fields; f0 += kMaxFields) {
    const int64_t nf = std::min<int64_t>(kMaxFields, num_fields - f0);
    FieldSet fs{};
    bool small_tables = true;  // every table below 2 GiB: the buffer-load kernel
    for (int64_t i = 0; i < nf; ++i) {
      fs.table[i] = tables[f0 + i];
      fs.rows[i] = table_rows[f0 + i];
      fs.div[i] = make_divisor(static_cast<uint64_t>(num_buckets[f0 + i]));
      small_tables = small_tables && table_rows[f0 + i] * dim * 4 < (int64_t(1) << 31);
    }
    if (small_tables) {
      // the pipelined kernel stores a run's 16 output rows through one
      // buffer resource (range < 2 GiB)
      if (lanes <= 4 && int64_t(kPipeBags) * ldo * 4 < (int64_t(1) << 31)) {
        // two runs per wave measured best on configs[3] (1 to 13 tried)
        const int64_t rpw = 2;
        if (combiner == ANNC_COMBINER_MEAN)
          launch_hashed_pipe<true>(fs, f0, nf, batch, dim, ids, offsets, out, ldo, buckets_out, rpw, s);
        else
          launch_hashed_pipe<false>(fs, f0, nf, batch, dim, ids, offsets, out, ldo, buckets_out, rpw, s);
      } else if (lanes <= 4)
        launch_hashed_wave_g<4>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
      else if (lanes <= 8)  // two bags per lane group: more positions hashed per wave
        launch_hashed_lds_g<8, 2>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
      else if (lanes <= 16)
        launch_hashed_lds_g<16, 2>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
      else if (lanes <= 32)
        launch_hashed_wave_g<32>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
      else
        launch_hashed_wave_g<64>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
      ANNC_HIP_TRY(hipGetLastError());
      continue;
    }
    if (lanes <= 4)
      launch_hashed_g<4>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
    else if (lanes <= 8)
      launch_hashed_g<8>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
    else if (lanes <= 16)
      launch_hashed_g<16>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
    else if (lanes <= 32)
      launch_hashed_g<32>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
    else
      launch_hashed_g<64>(fs, f0, nf, batch, dim, ids, offsets, combiner, out, ldo, buckets_out, s);
    ANNC_HIP_TRY(hipGetLastError());
  }
  return set_error(ANNC_OK, "");
}

}  // extern "C"

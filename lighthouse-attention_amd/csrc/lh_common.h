// Shared device/host helpers for the gfx950 Lighthouse kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lighthouse_hip.h"

#define LH_D 128  // head dimension supported by every kernel in this library

typedef uint16_t bf16_t;  // bfloat16 storage
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float floatx16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float floatx4 __attribute__((__vector_size__(4 * sizeof(float))));

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

// Two fp32 -> bf16 conversions in one v_cvt_pk_bf16_f32: round to nearest even
// (torch's bf16 cast), NaN stays NaN, no branches.
typedef float lh_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 lh_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const lh_f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, lh_bf16x2));
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return (bf16_t)(pack_bf16x2(f, 0.f) & 0xffffu); }

// 8 bf16 held in one 16-byte register quad.
__device__ __forceinline__ void unpack8(const uint4 v, float* f) {
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xffff0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xffff0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf16x2(f[0], f[1]); v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]); v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

// ---------------------------------------------------------------------------
// Element types of the row kernels (layer inputs, pyramid, attention rows and
// outputs): bf16, what the reference configs run, and fp16.  Both are 16-bit;
// arithmetic is fp32 with one rounding per stored value (round to nearest
// even, as torch's casts).  pack2(lo, hi) rounds two floats into one word,
// lo/hi widen the low/high half of a word.
// ---------------------------------------------------------------------------
typedef _Float16 lh_f16x2 __attribute__((ext_vector_type(2)));
struct BF16 {
  static constexpr int code = LH_DTYPE_BF16;
  __device__ static __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) { return pack_bf16x2(a, b); }
};
struct F16 {
  static constexpr int code = LH_DTYPE_F16;
  __device__ static __forceinline__ float lo(uint32_t w) { return (float)__builtin_bit_cast(lh_f16x2, w).x; }
  __device__ static __forceinline__ float hi(uint32_t w) { return (float)__builtin_bit_cast(lh_f16x2, w).y; }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    const lh_f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, lh_f16x2));
  }
};

// x rounded to the element type and widened back (a stored-then-loaded value)
template <typename T>
__device__ __forceinline__ float round_to(float x) { return T::lo(T::pack2(x, 0.f)); }

template <typename T>
__device__ __forceinline__ void unpack8_t(const uint4 v, float* f) {
  f[0] = T::lo(v.x); f[1] = T::hi(v.x); f[2] = T::lo(v.y); f[3] = T::hi(v.y);
  f[4] = T::lo(v.z); f[5] = T::hi(v.z); f[6] = T::lo(v.w); f[7] = T::hi(v.w);
}

template <typename T>
__device__ __forceinline__ uint4 pack8_t(const float* f) {
  uint4 v;
  v.x = T::pack2(f[0], f[1]); v.y = T::pack2(f[2], f[3]);
  v.z = T::pack2(f[4], f[5]); v.w = T::pack2(f[6], f[7]);
  return v;
}

// Launch helper: F(tag) for the element type named by a dtype code.
#define LH_DISPATCH_DTYPE(dtype, ...)                         \
  do {                                                       \
    if ((dtype) == LH_DTYPE_F16) {                           \
      using T = F16;                                         \
      __VA_ARGS__;                                           \
    } else {                                                 \
      using T = BF16;                                        \
      __VA_ARGS__;                                           \
    }                                                        \
  } while (0)

static inline bool valid_dtype(int dtype) { return dtype == LH_DTYPE_BF16 || dtype == LH_DTYPE_F16; }

// 16-byte store with the nontemporal hint (a vector store, `global_store ... nt`):
// for outputs that no kernel of the same pass reads back soon.  Their lines then
// do not stay dirty in the 256 MB last-level cache, where the next streaming
// kernel would have to write them back while it reads (pyramid backward ->
// next pyramid forward: 67 -> 53 us for the forward at cfg2, the backward
// 59 -> 68 us; fan-out 24.7 -> 23.0 us).
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store16_nt(void* p, const uint4 v) {
  __builtin_nontemporal_store(nt_u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2.
// Logical block of dispatch index w: each XCD gets a contiguous run, so
// neighbouring rows that read the same inputs (pooled rows shared by a span of
// tokens) share an L2.  Identity when the grid is not a multiple of 8.
// ---------------------------------------------------------------------------
__device__ __forceinline__ long long xcd_block(long long w, long long total) {
  return (total & 7) ? w : (w & 7) * (total >> 3) + (w >> 3);
}

// Runs of `run` consecutive blocks per XCD, the XCDs taking turns: dispatch
// index w (XCD w % 8) -> logical block, a bijection on [0, total) (the
// incomplete last group of 8 runs keeps the dispatch order).  Neighbouring
// blocks still share an L2, while every XCD sees the whole index range, so
// work that varies along it stays balanced across XCDs.
__device__ __forceinline__ long long xcd_run(long long w, long long total, int run) {
  const long long span = 8LL * run;
  const long long g = w / span;
  if ((g + 1) * span > total) return w;
  const long long r = w - g * span;
  return g * span + (r & 7) * run + (r >> 3);
}

// ---------------------------------------------------------------------------
// Rotary embedding of 8 consecutive elements of a row (pairs j = 0..3 are
// (f[2j], f[2j+1])) by the angles whose (cos, sin) pairs are c01 = (c0, s0, c1, s1)
// and c23 = (c2, s2, c3, s3).  FWD rotates by +theta (torchtitan's
// apply_rotary_emb: the complex product x * e^{i theta}), otherwise by -theta
// (its adjoint).  The fma placement is fixed here so every kernel that rotates
// produces the same bits.
// ---------------------------------------------------------------------------
template <bool FWD>
__device__ __forceinline__ void rope_rotate8(float* f, const float4 c01, const float4 c23) {
  const float c[4] = {c01.x, c01.z, c23.x, c23.z};
  const float s[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x0 = f[2 * j], x1 = f[2 * j + 1];
    if (FWD) {
      f[2 * j] = fmaf(x0, c[j], -(x1 * s[j]));
      f[2 * j + 1] = fmaf(x0, s[j], x1 * c[j]);
    } else {
      f[2 * j] = fmaf(x0, c[j], x1 * s[j]);
      f[2 * j + 1] = fmaf(x1, c[j], -(x0 * s[j]));
    }
  }
}

// (cos, sin) of the 4 pairs starting at element d0 (a multiple of 8) of position t,
// from a [.., D/2, 2] fp32 table
__device__ __forceinline__ void rope_freqs8(const float* fs, int64_t t, int D, int d0, float4& c01, float4& c23) {
  const float4* cs = reinterpret_cast<const float4*>(fs + (t * (D / 2) + d0 / 2) * 2);
  c01 = cs[0];
  c23 = cs[1];
}

// ---------------------------------------------------------------------------
// pyramid geometry (integer forms)
// ---------------------------------------------------------------------------
// Level l (1-based) has S / p^(l-1) nodes; levels are concatenated base first.
struct Pyramid {
  int S, L, p;
  int len[9];  // len[l] for l = 1..L
  int off[9];  // off[l] for l = 1..L
  int total;   // S_tot
};

static inline bool make_pyramid(int S, int L, int p, Pyramid* g) {
  if (S <= 0 || L < 1 || L > 8 || p < 2) return false;
  g->S = S; g->L = L; g->p = p;
  long long c = 1, acc = 0;
  for (int l = 1; l <= L; ++l) {
    g->len[l] = (int)(S / c);
    g->off[l] = (int)acc;
    acc += g->len[l];
    c *= p;
    if (c > (1LL << 30)) return false;
  }
  g->total = (int)acc;
  return true;
}

static inline int ipow(int b, int e) {
  int r = 1;
  for (int i = 0; i < e; ++i) r *= b;
  return r;
}

static inline int ilog2_exact(int p) {
  int s = 0;
  while ((1 << s) < p) ++s;
  return ((1 << s) == p) ? s : -1;
}

#define LH_CHECK_LAUNCH()                                  \
  do {                                                     \
    hipError_t _e = hipGetLastError();                     \
    if (_e != hipSuccess) return LH_ERR_LAUNCH;            \
  } while (0)

// Element-wise and row-wise kernels of the Llama3 block around the attention:
// rotary embedding fused with the q/k/v split of the projection output,
// RMSNorm forward/backward, SwiGLU forward/backward.  All are HBM-bound
// streaming passes: one 16-byte vector (8 bf16) per lane and access, every
// row read once; fp32 arithmetic, one rounding to bf16 per output.
#include "lh_common.h"

#include <mutex>

namespace {

constexpr int kVec = 8;  // bf16 per 16-byte access

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------------------
// rotary embedding on interleaved pairs (x[2j], x[2j+1]) by angle t * f_j:
//   forward  (a, b) -> (a c - b s, a s + b c)
//   backward (a, b) -> (a c + b s, b c - a s)      (rotation by -angle)
// cos/sin come from the caller's table fs[t][j] = (cos, sin), fp32.
// ---------------------------------------------------------------------------
struct RopeArgs {
  const bf16_t* x;       // fwd: projection output rows; bwd: unused
  const bf16_t* g[3];    // bwd: grads of q, k, v
  bf16_t* out[3];        // fwd: q, k, v contiguous [B, S, H, D]
  bf16_t* dx;            // bwd: projection-output grads
  const float* fs;       // [S, D/2, 2]
  int64_t xs;            // row stride of x / dx (elements)
  int64_t gsb[3], gss[3], gsh[3];  // bwd: strides of the three grads
  int S, Hq, Hkv, D;
  int64_t rows;          // B * S
  int chunks;            // 16-byte chunks per row = (Hq + 2 Hkv) * D / 8
};

template <bool FWD>
__global__ __launch_bounds__(256) void rope_qkv_kernel(const RopeArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.rows * a.chunks) return;
  const int64_t row = i / a.chunks;
  const int c = (int)(i - row * a.chunks);
  const int col = c * kVec;                 // element column inside the row
  const int head = col / a.D, d0 = col - head * a.D;
  const int which = head < a.Hq ? 0 : (head < a.Hq + a.Hkv ? 1 : 2);
  const int h = which == 0 ? head : (which == 1 ? head - a.Hq : head - a.Hq - a.Hkv);
  const int nh = which == 0 ? a.Hq : a.Hkv;
  const int b = (int)(row / a.S), t = (int)(row - (int64_t)b * a.S);
  uint4 in;
  if (FWD) {
    in = ld16(a.x + row * a.xs + col);
  } else {
    in = ld16(a.g[which] + b * a.gsb[which] + (int64_t)t * a.gss[which] + (int64_t)h * a.gsh[which] + d0);
  }
  uint4 o = in;
  if (which < 2) {
    float f[kVec];
    unpack8(in, f);
    float4 c01, c23;
    rope_freqs8(a.fs, t, a.D, d0, c01, c23);
    rope_rotate8<FWD>(f, c01, c23);
    o = pack8(f);
  }
  if (FWD) {
    st16(a.out[which] + ((row * nh + h) * a.D + d0), o);
  } else {
    st16(a.dx + row * a.xs + col, o);
  }
}

// ---------------------------------------------------------------------------
// RMSNorm: y = bf16((x * r) * w), r = 1 / sqrt(mean(x^2) + eps), fp32 inside.
// One wave per row; each lane holds up to 8 16-byte chunks (dim <= 4096, dim % 8 == 0).
// ---------------------------------------------------------------------------
constexpr int kMaxChunksPerLane = 8;  // dim <= 64 * 8 * 8 = 4096

// With a residual input res (ADD): h = bf16(x + res) is written out and normalised.
template <int NC, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ res,
                                                          const bf16_t* __restrict__ w, bf16_t* __restrict__ h,
                                                          bf16_t* __restrict__ y, float* __restrict__ rstd,
                                                          int64_t rows, int dim, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bf16_t* xr = x + row * dim;
  float v[NC][kVec];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = (c * 64 + lane) * kVec;
    unpack8(col < dim ? ld16(xr + col) : make_uint4(0, 0, 0, 0), v[c]);
    if (ADD && col < dim) {
      float rv[kVec];
      unpack8(ld16(res + row * dim + col), rv);
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[c][e] += rv[e];
      const uint4 hv = pack8(v[c]);
      st16(h + row * dim + col, hv);
      unpack8(hv, v[c]);  // normalise the rounded sum, as a separate norm of h would
    }
#pragma unroll
    for (int e = 0; e < kVec; ++e) ss += v[c][e] * v[c][e];
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)dim + eps);
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = (c * 64 + lane) * kVec;
    if (col < dim) {
      float wf[kVec];
      unpack8(ld16(w + col), wf);
#pragma unroll
      for (int e = 0; e < kVec; ++e) v[c][e] = (v[c][e] * r) * wf[e];
      st16(y + row * dim + col, pack8(v[c]));
    }
  }
}

// dx = r * g - x * r^3 * mean(g * x), g = dy * w;  dw = sum over rows of dy * x * r.
// Block = 4 waves over a contiguous range of rows; each block leaves one fp32
// partial of every dw column (stored column-major, [dim][blocks]) for
// rmsnorm_dw_kernel.
// one row's dy, x and (if given) dres slices of this lane
template <int NC>
__device__ __forceinline__ void rms_bwd_load(const bf16_t* __restrict__ dy, const bf16_t* __restrict__ x,
                                             const bf16_t* __restrict__ dres, int64_t row, int dim, int lane,
                                             uint4 (&a)[NC], uint4 (&b)[NC], uint4 (&c2)[NC]) {
  const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = (c * 64 + lane) * kVec;
    a[c] = col < dim ? ld16(dy + row * dim + col) : zero;
    b[c] = col < dim ? ld16(x + row * dim + col) : zero;
    c2[c] = (dres && col < dim) ? ld16(dres + row * dim + col) : zero;
  }
}

template <int NC>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const bf16_t* __restrict__ dy, const bf16_t* __restrict__ x,
                                                          const bf16_t* __restrict__ w, const float* __restrict__ rstd,
                                                          const bf16_t* __restrict__ dres, bf16_t* __restrict__ dx,
                                                          float* __restrict__ dw_part, int64_t rows, int dim,
                                                          int64_t rows_per_block) {
  // waves 1..3 hand their dw partials to wave 0, half of the lane's chunks at a time
  __shared__ float red[3][64 * kVec * kMaxChunksPerLane / 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = min(rows, r0 + rows_per_block);
  float wf[NC][kVec], acc[NC][kVec];
  const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int col = (c * 64 + lane) * kVec;
    unpack8(col < dim ? ld16(w + col) : zero, wf[c]);
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[c][e] = 0.f;
  }
  // Each wave walks every fourth row of the block; the next row's dy, x (and
  // dres) are loaded before this row's reduction, so a row's memory latency
  // overlaps the previous row's work.
  uint4 cd[NC], cx[NC], cr[NC];
  if (r0 + wave < r1) rms_bwd_load<NC>(dy, x, dres, r0 + wave, dim, lane, cd, cx, cr);
  for (int64_t row = r0 + wave; row < r1; row += 4) {
    float g[NC][kVec], xv[NC][kVec], d[NC][kVec];
    uint4 nd[NC], nx[NC], nr[NC];
    if (row + 4 < r1) rms_bwd_load<NC>(dy, x, dres, row + 4, dim, lane, nd, nx, nr);
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      unpack8(cd[c], d[c]);
      unpack8(cx[c], xv[c]);
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        g[c][e] = d[c][e] * wf[c][e];
        dot += g[c][e] * xv[c][e];
      }
    }
    dot = wave_sum(dot);
    const float r = rstd[row];
    const float k3 = r * r * r * dot / (float)dim;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int e = 0; e < kVec; ++e) {
        acc[c][e] += d[c][e] * (xv[c][e] * r);
        g[c][e] = r * g[c][e] - xv[c][e] * k3;
      }
      const int col = (c * 64 + lane) * kVec;
      if (col < dim) {
        if (dres) {  // gradient arriving through the residual branch, summed before one rounding
          float rv[kVec];
          unpack8(cr[c], rv);
#pragma unroll
          for (int e = 0; e < kVec; ++e) g[c][e] += rv[e];
        }
        st16(dx + row * dim + col, pack8(g[c]));
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      cd[c] = nd[c];
      cx[c] = nx[c];
      cr[c] = nr[c];
    }
  }
  // reduce the four waves' dw partials through LDS, NC chunks at a time in halves
  float* red0 = &red[0][0];
  constexpr int HALF = (NC + 1) / 2;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int cb = part * HALF, ce = min(NC, cb + HALF);
    if (wave > 0) {
      for (int c = cb; c < ce; ++c)
#pragma unroll
        for (int e = 0; e < kVec; ++e)
          red0[(wave - 1) * (64 * kVec * kMaxChunksPerLane / 2) + ((c - cb) * 64 + lane) * kVec + e] = acc[c][e];
    }
    __syncthreads();
    if (wave == 0) {
      for (int c = cb; c < ce; ++c) {
#pragma unroll
        for (int e = 0; e < kVec; ++e) {
          float s = acc[c][e];
#pragma unroll
          for (int q = 0; q < 3; ++q) s += red0[q * (64 * kVec * kMaxChunksPerLane / 2) + ((c - cb) * 64 + lane) * kVec + e];
          if ((c * 64 + lane) * kVec < dim) dw_part[(int64_t)((c * 64 + lane) * kVec + e) * gridDim.x + blockIdx.x] = s;
        }
      }
    }
    __syncthreads();
  }
}

// dw[i] = sum of column i's partials: one wave per column, lanes stride the
// contiguous partials, then a wave reduction (fixed order: deterministic).
__global__ __launch_bounds__(256) void rmsnorm_dw_kernel(const float* __restrict__ part, bf16_t* __restrict__ dw,
                                                         int parts, int dim) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= dim) return;
  const float* col = part + (int64_t)i * parts;
  float s = 0.f;
  for (int p = lane; p < parts; p += 64) s += col[p];
  s = wave_sum(s);
  if (lane == 0) dw[i] = f32_to_bf16(s);
}

// ---------------------------------------------------------------------------
// SwiGLU on the fused [h1 | h3] projection output (row length 2F):
//   a = bf16(bf16(silu(h1)) * h3)
//   backward: dh3 = bf16(da * bf16(silu(h1))),
//             dh1 = bf16(bf16(da * h3) * sigmoid(h1) * (1 + h1 (1 - sigmoid(h1))))
// (the roundings of torch's separate silu and mul ops, in the same order).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

template <bool FWD>
__global__ __launch_bounds__(256) void swiglu_kernel(const bf16_t* __restrict__ h, const bf16_t* __restrict__ da,
                                                     bf16_t* __restrict__ out, int64_t rows, int F) {
  const int cpr = F / kVec;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * cpr) return;
  const int64_t row = i / cpr;
  const int col = (int)(i - row * cpr) * kVec;
  float h1[kVec], h3[kVec];
  unpack8(ld16(h + row * 2 * F + col), h1);
  unpack8(ld16(h + row * 2 * F + F + col), h3);
  if (FWD) {
    float a[kVec];
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      const float s = bf16_round(h1[e] / (1.0f + expf(-h1[e])));
      a[e] = s * h3[e];
    }
    st16(out + row * F + col, pack8(a));
  } else {
    float g[kVec], d1[kVec], d3[kVec];
    unpack8(ld16(da + row * F + col), g);
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      const float sg = 1.0f / (1.0f + expf(-h1[e]));
      const float s = bf16_round(h1[e] / (1.0f + expf(-h1[e])));
      d3[e] = g[e] * s;
      const float gs = bf16_round(g[e] * h3[e]);
      d1[e] = gs * sg * (1.0f + h1[e] * (1.0f - sg));
    }
    st16(out + row * 2 * F + col, pack8(d1));
    st16(out + row * 2 * F + F + col, pack8(d3));
  }
}

// ---------------------------------------------------------------------------
// Split-K weight gradient: out[i] = bf16(sum over s of part[s][i]), fp32 sum in
// slice order (what one accumulation over the whole token axis would give up
// to fp32 reassociation), 8 outputs per lane.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ part, bf16_t* __restrict__ out,
                                                         int splits, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * kVec;
  if (i >= n) return;
  float acc[kVec] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int sp = 0; sp < splits; ++sp) {
    const float4* p = reinterpret_cast<const float4*>(part + (int64_t)sp * n + i);
    const float4 a = p[0], b = p[1];
    acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
    acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
  }
  st16(out + i, pack8(acc));
}

inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

inline int grid_of(int64_t n) { return (int)((n + 255) / 256); }

}  // namespace

extern "C" int lh_rope_qkv_fwd(const void* x, int64_t xs, const float* freqs, void* q, void* k, void* v,
                               int B, int S, int Hq, int Hkv, int D, void* stream) {
  if (!x || !freqs || !q || !k || !v || B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0) return LH_ERR_INVALID_ARG;
  if (D % 8 || xs < (int64_t)(Hq + 2 * Hkv) * D || xs % 8 || !al16(x) || !al16(q) || !al16(k) || !al16(v) ||
      !al16(freqs))
    return LH_ERR_INVALID_ARG;
  RopeArgs a{};
  a.x = (const bf16_t*)x;
  a.out[0] = (bf16_t*)q; a.out[1] = (bf16_t*)k; a.out[2] = (bf16_t*)v;
  a.fs = freqs; a.xs = xs; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.D = D;
  a.rows = (int64_t)B * S;
  a.chunks = (Hq + 2 * Hkv) * D / kVec;
  const int64_t n = a.rows * a.chunks;
  if (n / 256 + 1 > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
  rope_qkv_kernel<true><<<grid_of(n), 256, 0, (hipStream_t)stream>>>(a);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

extern "C" int lh_rope_qkv_bwd(const void* dq, const void* dk, const void* dv, const int64_t* strides,
                               const float* freqs, void* dx, int64_t xs, int B, int S, int Hq, int Hkv, int D,
                               void* stream) {
  if (!dq || !dk || !dv || !strides || !freqs || !dx || B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0)
    return LH_ERR_INVALID_ARG;
  if (D % 8 || xs < (int64_t)(Hq + 2 * Hkv) * D || xs % 8 || !al16(dq) || !al16(dk) || !al16(dv) || !al16(dx) ||
      !al16(freqs))
    return LH_ERR_INVALID_ARG;
  RopeArgs a{};
  a.g[0] = (const bf16_t*)dq; a.g[1] = (const bf16_t*)dk; a.g[2] = (const bf16_t*)dv;
  for (int i = 0; i < 3; ++i) {
    a.gsb[i] = strides[3 * i]; a.gss[i] = strides[3 * i + 1]; a.gsh[i] = strides[3 * i + 2];
    if ((a.gsb[i] | a.gss[i] | a.gsh[i]) % 8) return LH_ERR_INVALID_ARG;
  }
  a.dx = (bf16_t*)dx; a.fs = freqs; a.xs = xs; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.D = D;
  a.rows = (int64_t)B * S;
  a.chunks = (Hq + 2 * Hkv) * D / kVec;
  const int64_t n = a.rows * a.chunks;
  if (n / 256 + 1 > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
  rope_qkv_kernel<false><<<grid_of(n), 256, 0, (hipStream_t)stream>>>(a);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

#define LH_NC_DISPATCH(NCV, CALL) \
  switch (NCV) {                  \
    case 1: { constexpr int NC = 1; CALL; break; } \
    case 2: { constexpr int NC = 2; CALL; break; } \
    case 3: { constexpr int NC = 3; CALL; break; } \
    case 4: { constexpr int NC = 4; CALL; break; } \
    case 5: { constexpr int NC = 5; CALL; break; } \
    case 6: { constexpr int NC = 6; CALL; break; } \
    case 7: { constexpr int NC = 7; CALL; break; } \
    case 8: { constexpr int NC = 8; CALL; break; } \
    default: return LH_ERR_UNSUPPORTED;            \
  }

extern "C" int lh_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows, int dim, float eps,
                              void* stream) {
  if (!x || !w || !y || !rstd || rows <= 0 || dim <= 0 || !(eps >= 0.f)) return LH_ERR_INVALID_ARG;
  if (!al16(x) || !al16(w) || !al16(y)) return LH_ERR_INVALID_ARG;
  if (dim % 8 || dim > 4096) return LH_ERR_UNSUPPORTED;  // whole 16-byte chunks, <= 8 per lane
  const int nc = (dim + 511) / 512;
  const int grid = (int)((rows + 3) / 4);
  LH_NC_DISPATCH(nc, (rmsnorm_fwd_kernel<NC, false><<<grid, 256, 0, (hipStream_t)stream>>>(
                          (const bf16_t*)x, nullptr, (const bf16_t*)w, nullptr, (bf16_t*)y, rstd, rows, dim, eps)));
  LH_CHECK_LAUNCH();
  return LH_OK;
}

extern "C" int lh_add_rmsnorm_fwd(const void* x, const void* r, const void* w, void* h, void* y, float* rstd,
                                  int64_t rows, int dim, float eps, void* stream) {
  if (!x || !r || !w || !h || !y || !rstd || rows <= 0 || dim <= 0 || !(eps >= 0.f)) return LH_ERR_INVALID_ARG;
  if (!al16(x) || !al16(r) || !al16(w) || !al16(h) || !al16(y)) return LH_ERR_INVALID_ARG;
  if (dim % 8 || dim > 4096) return LH_ERR_UNSUPPORTED;
  const int nc = (dim + 511) / 512;
  const int grid = (int)((rows + 3) / 4);
  LH_NC_DISPATCH(nc, (rmsnorm_fwd_kernel<NC, true><<<grid, 256, 0, (hipStream_t)stream>>>(
                          (const bf16_t*)x, (const bf16_t*)r, (const bf16_t*)w, (bf16_t*)h, (bf16_t*)y, rstd, rows,
                          dim, eps)));
  LH_CHECK_LAUNCH();
  return LH_OK;
}

extern "C" int lh_rmsnorm_bwd(const void* dy, const void* x, const void* w, const float* rstd, const void* dres,
                              void* dx, void* dw, float* dw_part, int parts, int64_t rows, int dim, void* stream) {
  if (!dy || !x || !w || !rstd || !dx || !dw || !dw_part || rows <= 0 || dim <= 0 || parts <= 0)
    return LH_ERR_INVALID_ARG;
  if (!al16(dy) || !al16(x) || !al16(w) || !al16(dx) || (dres && !al16(dres))) return LH_ERR_INVALID_ARG;
  if (dim % 8 || dim > 4096) return LH_ERR_UNSUPPORTED;
  const int nc = (dim + 511) / 512;
  const int64_t rpb = (rows + parts - 1) / parts;
  const int used = (int)((rows + rpb - 1) / rpb);  // blocks that own at least one row
  LH_NC_DISPATCH(nc, (rmsnorm_bwd_kernel<NC><<<used, 256, 0, (hipStream_t)stream>>>(
                          (const bf16_t*)dy, (const bf16_t*)x, (const bf16_t*)w, rstd, (const bf16_t*)dres,
                          (bf16_t*)dx, dw_part, rows, dim, rpb)));
  LH_CHECK_LAUNCH();
  rmsnorm_dw_kernel<<<(dim + 3) / 4, 256, 0, (hipStream_t)stream>>>(dw_part, (bf16_t*)dw, used, dim);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

// ---------------------------------------------------------------------------
// RMSNorm backward without a caller workspace: the dw partials live in a
// file-scope device array (one copy per GPU, held until the process ends).
// Its device address is looked up once per device with hipGetSymbolAddress;
// in host code the array's name is only a host-side stand-in.  Every launch
// writes each partial it later reads, so nothing needs clearing.  Calls that
// overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
constexpr int kNoAllocParts = 256;
constexpr int kNoAllocMaxDim = 4096;
static __device__ __align__(256) float scratch[kNoAllocParts * kNoAllocMaxDim];  // 4 MiB

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int scratch_on_current_device(float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return LH_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LH_ERR_LAUNCH;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return LH_OK;
}
}  // namespace

extern "C" int lh_rmsnorm_bwd_noalloc(const void* dy, const void* x, const void* w, const float* rstd,
                                      const void* dres, void* dx, void* dw, int64_t rows, int dim, void* stream) {
  if (!dy || !x || !w || !rstd || !dx || !dw || rows <= 0 || dim <= 0) return LH_ERR_INVALID_ARG;
  if (dim > kNoAllocMaxDim) return LH_ERR_UNSUPPORTED;
  float* part = nullptr;
  const int rc = scratch_on_current_device(&part);
  if (rc != LH_OK) return rc;
  return lh_rmsnorm_bwd(dy, x, w, rstd, dres, dx, dw, part, kNoAllocParts, rows, dim, stream);
}

extern "C" int lh_swiglu_fwd(const void* h, void* a, int64_t rows, int F, void* stream) {
  if (!h || !a || rows <= 0 || F <= 0 || F % 8 || !al16(h) || !al16(a)) return LH_ERR_INVALID_ARG;
  const int64_t n = rows * (F / kVec);
  if (n / 256 + 1 > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
  swiglu_kernel<true><<<grid_of(n), 256, 0, (hipStream_t)stream>>>((const bf16_t*)h, nullptr, (bf16_t*)a, rows, F);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

extern "C" int lh_swiglu_bwd(const void* da, const void* h, void* dh, int64_t rows, int F, void* stream) {
  if (!da || !h || !dh || rows <= 0 || F <= 0 || F % 8 || !al16(h) || !al16(da) || !al16(dh))
    return LH_ERR_INVALID_ARG;
  const int64_t n = rows * (F / kVec);
  if (n / 256 + 1 > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
  swiglu_kernel<false><<<grid_of(n), 256, 0, (hipStream_t)stream>>>((const bf16_t*)h, (const bf16_t*)da, (bf16_t*)dh,
                                                                     rows, F);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

extern "C" int lh_splitk_sum(const float* part, void* out, int splits, int64_t n, void* stream) {
  if (!part || !out || splits <= 0 || n <= 0 || n % 8 || !al16(part) || !al16(out)) return LH_ERR_INVALID_ARG;
  const int64_t threads = n / kVec;
  if (threads / 256 + 1 > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
  splitk_sum_kernel<<<grid_of(threads), 256, 0, (hipStream_t)stream>>>(part, (bf16_t*)out, splits, n);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

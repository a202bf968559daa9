// Fan-out of selected rows onto the base sequence (forward) and its adjoint.
//
// Forward restates _scatter_fanout_fwd_kernel (src/lighthouse_selection.py:408-459):
// the entry at level l, local index i, is added to base positions
// [(i+1)c_l - 1, (i+2)c_l - 2].  Turned around, base position t receives, from
// each level, the node floor((t+1)/c_l) - 1 if that node was selected.  Each
// output row therefore gathers at most L rows through the inverse map, sums in
// fp32 and rounds once: no zero-fill, no atomics, deterministic.
//
// Backward restates _scatter_fanout_bwd_kernel (:462-514): each selected row
// sums dout over its span.  The same pass forms delta = rowsum(dattn * o) for
// the attention backward from the rounded dattn, as SDPA's backward does.
// Rows are bf16 or fp16 (the element type T), sums fp32.
#include "lh_common.h"

namespace {

struct ScatArgs {
  const bf16_t* src;       // fwd: attn [BH, n, D];  bwd: dout, [b, h, t] at b*sb + h*sh + t*st
  const int32_t* map;      // fwd: inverse [BH, S_tot];  bwd: indices [BH, n]
  const bf16_t* o;         // bwd: attention output [BH, n, D] (optional)
  bf16_t* dst;             // fwd: out, [b, h, t] at b*sb + h*sh + t*st;  bwd: dattn [BH, n, D]
  float* delta;            // bwd: [BH, n] (optional)
  int64_t sb, sh, st;      // element strides of the base-sequence tensor (D contiguous)
  int H, S, S_out, n, L, shift, S_tot;
  int off[9], len[9];
  long long rows;
};

__device__ __forceinline__ uint4 ld16(const bf16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Both kernels take their block index through xcd_run: consecutive blocks
// share rows (neighbouring base tokens read the same selected rows; a node's
// span overlaps its descendants', which precede it in causal order), and
// workgroups are dispatched round-robin over the 8 XCDs, each with its own L2,
// so runs of SCAT_RUN consecutive blocks are kept on one XCD.  Short runs
// rather than one contiguous eighth per XCD: an eighth is one head here, and the
// span lengths (the adjoint's work) differ from head to head.
constexpr int SCAT_RUN = 16;
//
// Forward: each 16-lane group owns SF_ROWS output rows (16 apart); all their
// levels' inverse lookups are issued first, then all row loads, so a group
// has SF_ROWS * NL loads in flight across two dependent round trips.
constexpr int SF_ROWS = 2;
template <typename T, int NL, int R>
__global__ __launch_bounds__(256) void scatter_fwd_kernel(const ScatArgs a) {
  const int tid = threadIdx.x;
  const int l16 = tid & 15;
  const long long row0 = xcd_run(blockIdx.x, gridDim.x, SCAT_RUN) * (16 * R) + (tid >> 4);
  int s[R][NL], tr[R];
  long long bhr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long long row = row0 + 16 * r;
    const bool ok = row < a.rows;
    const long long bh = ok ? row / a.S_out : 0;
    const int t = ok ? (int)(row - bh * a.S_out) : 0;
    tr[r] = ok ? t : -1;
    bhr[r] = bh;
    const int32_t* inv = a.map + bh * a.S_tot;
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      const int node = ((t + 1) >> (l * a.shift)) - 1;
      s[r][l] = (ok && node >= 0 && node < a.len[l + 1]) ? inv[a.off[l + 1] + node] : -1;
    }
  }
  uint4 v[R][NL];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bf16_t* src = a.src + (size_t)bhr[r] * a.n * LH_D + 8 * l16;
#pragma unroll
    for (int l = 0; l < NL; ++l)
      v[r][l] = s[r][l] >= 0 ? ld16(src + (size_t)s[r][l] * LH_D) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (tr[r] < 0) continue;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      if (s[r][l] < 0) continue;  // keeps the fp32 sum of exactly the present terms
      float f[8];
      unpack8_t<T>(v[r][l], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += f[e];
    }
    const int b = (int)(bhr[r] / a.H), h = (int)(bhr[r] % a.H);
    store16_nt(a.dst + b * a.sb + h * a.sh + (int64_t)tr[r] * a.st + 8 * l16, pack8_t<T>(acc));
  }
}

// Backward: the span's dout rows are loaded eight at a time (independent
// loads), and the attention-output row for delta is loaded up front.  A block
// is one wave (4 rows; spans of 1 to p^(L-1) rows make waves finish at
// different times, and one-wave blocks free their slots soonest); XCD runs
// stay 256 rows long.
constexpr int SB_ROWS = 4;
template <typename T>
__global__ __launch_bounds__(16 * SB_ROWS) void scatter_bwd_kernel(const ScatArgs a) {
  const int tid = threadIdx.x;
  const long long row = xcd_run(blockIdx.x, gridDim.x, SCAT_RUN * 16 / SB_ROWS) * SB_ROWS + (tid >> 4);
  const int l16 = tid & 15;
  if (row >= a.rows) return;  // all 16 lanes of a row leave together
  const long long bh = row / a.n;
  const int r = a.map[row];
  uint4 ov = make_uint4(0, 0, 0, 0);
  if (a.delta) ov = ld16(a.o + (size_t)row * LH_D + 8 * l16);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (r >= 0 && r < a.S_tot) {
    int lvl = 1;
    while (lvl < a.L && r >= a.off[lvl + 1]) ++lvl;
    const int cs = (lvl - 1) * a.shift;
    const int c = 1 << cs;
    const int local = r - a.off[lvl];
    const int start = local * c + c - 1;
    const int stop = min(start + c, a.S_out);
    const int b = (int)(bh / a.H), h = (int)(bh % a.H);
    const bf16_t* src = a.src + b * a.sb + h * a.sh + 8 * l16;
    for (int t = start; t < stop; t += 8) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = t + u < stop ? ld16(src + (t + u) * a.st) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (t + u >= stop) break;  // same left-to-right fp32 sum as one row at a time
        float f[8];
        unpack8_t<T>(v[u], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += f[e];
      }
    }
  }
  const uint4 packed = pack8_t<T>(acc);
  *reinterpret_cast<uint4*>(a.dst + (size_t)row * LH_D + 8 * l16) = packed;
  if (a.delta) {
    float g[8], o[8];
    unpack8_t<T>(packed, g);
    unpack8_t<T>(ov, o);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d = fmaf(g[e], o[e], d);
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) d += __shfl_xor(d, m, 16);
    if (l16 == 0) a.delta[row] = d;
  }
}

int fill(ScatArgs& a, int S, int S_out, int n, int L, int p, int B, int H, int64_t sb, int64_t sh, int64_t st) {
  const int shift = ilog2_exact(p);
  if (shift <= 0 || L < 1 || L > 8 || S <= 0 || S_out <= 0 || n < 0 || B <= 0 || H <= 0) return LH_ERR_INVALID_ARG;
  if ((sb | sh | st) % 8 || sb < 0 || sh < 0 || st <= 0) return LH_ERR_INVALID_ARG;
  Pyramid g;
  if (!make_pyramid(S, L, p, &g)) return LH_ERR_INVALID_ARG;
  a.sb = sb; a.sh = sh; a.st = st; a.H = H;
  a.S = S; a.S_out = S_out; a.n = n; a.L = L; a.shift = shift; a.S_tot = g.total;
  for (int l = 1; l <= L; ++l) { a.off[l] = g.off[l]; a.len[l] = g.len[l]; }
  return LH_OK;
}

}  // namespace

extern "C" int lh_scatter_fwd(const void* attn, const int32_t* inverse, void* out, int64_t ob, int64_t oh,
                              int64_t os, int B, int H, int S, int S_out, int n, int D, int L, int p, int dtype,
                              void* stream) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!attn || !inverse || !out || ((uintptr_t)out & 15) || !valid_dtype(dtype)) return LH_ERR_INVALID_ARG;
  ScatArgs a{};
  int rc = fill(a, S, S_out, n, L, p, B, H, ob, oh, os);
  if (rc) return rc;
  a.src = (const bf16_t*)attn; a.map = inverse; a.dst = (bf16_t*)out;
  a.rows = (long long)B * H * S_out;
  const long long blocks = (a.rows + 16 * SF_ROWS - 1) / (16 * SF_ROWS);
  if (blocks > 2147483647LL) return LH_ERR_UNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)blocks), blk(256);
  LH_DISPATCH_DTYPE(dtype, switch (L) {
    case 1: hipLaunchKernelGGL((scatter_fwd_kernel<T, 1, SF_ROWS>), grid, blk, 0, st, a); break;
    case 2: hipLaunchKernelGGL((scatter_fwd_kernel<T, 2, SF_ROWS>), grid, blk, 0, st, a); break;
    case 3: hipLaunchKernelGGL((scatter_fwd_kernel<T, 3, SF_ROWS>), grid, blk, 0, st, a); break;
    case 4: hipLaunchKernelGGL((scatter_fwd_kernel<T, 4, SF_ROWS>), grid, blk, 0, st, a); break;
    case 5: hipLaunchKernelGGL((scatter_fwd_kernel<T, 5, SF_ROWS>), grid, blk, 0, st, a); break;
    case 6: hipLaunchKernelGGL((scatter_fwd_kernel<T, 6, SF_ROWS>), grid, blk, 0, st, a); break;
    case 7: hipLaunchKernelGGL((scatter_fwd_kernel<T, 7, SF_ROWS>), grid, blk, 0, st, a); break;
    default: hipLaunchKernelGGL((scatter_fwd_kernel<T, 8, SF_ROWS>), grid, blk, 0, st, a); break;
  });
  LH_CHECK_LAUNCH();
  return LH_OK;
}

extern "C" int lh_scatter_bwd(const void* dout, int64_t db, int64_t dh, int64_t ds, const int32_t* indices,
                              const void* o, void* dattn, float* delta, int B, int H, int S, int S_out, int n, int D,
                              int L, int p, int dtype, void* stream) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!dout || !indices || !dattn || ((o == nullptr) != (delta == nullptr)) || ((uintptr_t)dout & 15) ||
      !valid_dtype(dtype))
    return LH_ERR_INVALID_ARG;
  ScatArgs a{};
  int rc = fill(a, S, S_out, n, L, p, B, H, db, dh, ds);
  if (rc) return rc;
  a.src = (const bf16_t*)dout; a.map = indices; a.o = (const bf16_t*)o; a.dst = (bf16_t*)dattn; a.delta = delta;
  a.rows = (long long)B * H * n;
  if (a.rows == 0) return LH_OK;
  const long long blocks = (a.rows + SB_ROWS - 1) / SB_ROWS;
  if (blocks > 2147483647LL) return LH_ERR_UNSUPPORTED;
  LH_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL(scatter_bwd_kernel<T>, dim3((unsigned)blocks), dim3(16 * SB_ROWS), 0,
                                              reinterpret_cast<hipStream_t>(stream), a));
  LH_CHECK_LAUNCH();
  return LH_OK;
}

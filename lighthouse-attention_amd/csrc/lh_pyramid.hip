// Norm scorer + mean-pooled Q/K/V pyramid (forward) and the pyramid backward.
//
// Forward restates DialatedLighthouseNormScorer.forward
// (src/lighthouse_selection.py:589-616): base scores are the L2 norms of q and
// k rows, rounded to the row type (bf16 or fp16) like torch's `norm` of such
// rows; level j = 1..L-1 rows are
// the means of p^j consecutive base rows (fp32 sum, one rounding), and level-j
// scores are maxima of the base scores over the same span.  One pass streams
// xq/xk/xv once: 16 lanes own one (b, span, head) unit, 8 bf16 each, and walk
// the p^(L-1) base tokens of the span.  Base rows are never copied: pooled rows
// go to a separate [B, Sp, H, D] buffer.
//
// Backward restates the autograd of gather + cat + mean: each base row gets
// its own selected-space gradient plus, for every pooled level that contains
// it, that node's gradient / c_l.  Gather-formulated through the inverse map,
// so there are no atomics and the result is deterministic.
#include "lh_common.h"

namespace {

struct PyrArgs {
  const bf16_t *xq, *xk, *xv;
  int64_t sb, ss, sh;
  bf16_t *pq, *pk, *pv;
  int64_t pb, ps, ph;
  float *sqk, *skq;
  const float* fs;   // rotary (cos, sin) table [>= S, D/2, 2] (ROPE)
  bf16_t *rq, *rk;   // rotated base rows out (ROPE)
  int64_t rb, rs, rh;
  int B, S, H, L, shift, S_tot, nspan, cmax, units;
  int off[9], len[9];
};

__device__ __forceinline__ uint4 ld16(const bf16_t* p) { return *reinterpret_cast<const uint4*>(p); }

constexpr int PYR_CHUNK = 4;  // base tokens whose loads are issued together

// One base token t of (b, h): unpack the 16-byte slices of its q, k, v rows,
// rotate q and k (ROPE: rounded to bf16 and stored to rq / rk, the rounded
// values kept), and make its base scores: the bf16-rounded L2 norms of q and k
// (every lane of the 16-lane group gets them), or the given ones (GIVEN: sq, sk
// on entry).
template <typename T, bool GIVEN, bool ROPE>
__device__ __forceinline__ void pyr_token(const PyrArgs& a, int b, int h, int l16, size_t srow, int t,
                                          const uint4 xq, const uint4 xk, const uint4 xv, float* fq, float* fk,
                                          float* fv, float& sq, float& sk) {
  unpack8_t<T>(xq, fq);
  unpack8_t<T>(xk, fk);
  unpack8_t<T>(xv, fv);
  if (ROPE) {
    float4 c01, c23;
    rope_freqs8(a.fs, t, LH_D, 8 * l16, c01, c23);
    rope_rotate8<true>(fq, c01, c23);
    rope_rotate8<true>(fk, c01, c23);
    const uint4 wq = pack8_t<T>(fq), wk = pack8_t<T>(fk);
    const int64_t ro = (int64_t)b * a.rb + (int64_t)t * a.rs + (int64_t)h * a.rh + 8 * l16;
    *reinterpret_cast<uint4*>(a.rq + ro) = wq;
    *reinterpret_cast<uint4*>(a.rk + ro) = wk;
    unpack8_t<T>(wq, fq);
    unpack8_t<T>(wk, fk);
  }
  if (!GIVEN) {
    float pq = 0.f, pk = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) { pq = fmaf(fq[e], fq[e], pq); pk = fmaf(fk[e], fk[e], pk); }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) { pq += __shfl_xor(pq, m, 16); pk += __shfl_xor(pk, m, 16); }
    sq = round_to<T>(sqrtf(pq));
    sk = round_to<T>(sqrtf(pk));
  }
}

// ROPE: xq / xk are the projection's unrotated rows; each is rotated by its
// position's angles, rounded to bf16 and written to rq / rk, and the norms and
// means below are taken of those rounded rows, exactly as if the rotated rows
// had been stored first and read back.
template <typename T, int NL, bool GIVEN, bool ROPE>
__global__ __launch_bounds__(256) void pyramid_fwd_kernel(const PyrArgs a) {
  const int tid = threadIdx.x;
  const int u = blockIdx.x * 16 + (tid >> 4);
  const int l16 = tid & 15;
  if (u >= a.units) return;
  const int h = u % a.H;
  const int rest = u / a.H;
  const int span = rest % a.nspan;
  const int b = rest / a.nspan;
  const int t0 = span * a.cmax;
  const int t1 = min(a.S, t0 + a.cmax);
  const size_t srow = (size_t)(b * a.H + h) * a.S_tot;

  constexpr int NA = NL > 0 ? NL : 1;
  float accq[NA][8], acck[NA][8], accv[NA][8], mq[NA], mk[NA];
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    mq[l] = -INFINITY; mk[l] = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) { accq[l][e] = 0.f; acck[l][e] = 0.f; accv[l][e] = 0.f; }
  }
  const int64_t xoff = (int64_t)b * a.sb + (int64_t)h * a.sh + 8 * l16;
  float bq = 0.f, bk = 0.f;  // this lane's pending base scores
  // one base token: rows (q, k, v) as loaded, base scores when GIVEN
  auto token = [&](int t, const uint4 xq, const uint4 xk, const uint4 xv, float sq, float sk)
      __attribute__((always_inline)) {
    float fq[8], fk[8], fv[8];
    pyr_token<T, GIVEN, ROPE>(a, b, h, l16, srow, t, xq, xk, xv, fq, fk, fv, sq, sk);
    if (!GIVEN) {
      // base scores leave 16 tokens at a time: lane j keeps token t0 + 16 i + j,
      // and the group stores them as one contiguous 64-byte run per tensor
      const int j = (t - t0) & 15;
      if (l16 == j) { bq = sq; bk = sk; }
      if ((j == 15 || t == t1 - 1) && l16 <= j) {
        a.sqk[srow + t - j + l16] = bq;
        a.skq[srow + t - j + l16] = bk;
      }
    }
#pragma unroll
    for (int l = 0; l < NL; ++l) {
#pragma unroll
      for (int e = 0; e < 8; ++e) { accq[l][e] += fq[e]; acck[l][e] += fk[e]; accv[l][e] += fv[e]; }
      mq[l] = fmaxf(mq[l], sq);
      mk[l] = fmaxf(mk[l], sk);
      const int cs = (l + 1) * a.shift;  // log2 of the span of level l+2
      if (((t + 1) & ((1 << cs) - 1)) == 0) {
        const int node = t >> cs;
        const int lvl = l + 2;
        const float inv_c = 1.0f / (float)(1 << cs);
        float mo[8];
        const int64_t prow = (int64_t)b * a.pb + (int64_t)(a.off[lvl] - a.S + node) * a.ps + (int64_t)h * a.ph + 8 * l16;
#pragma unroll
        for (int e = 0; e < 8; ++e) mo[e] = accq[l][e] * inv_c;
        *reinterpret_cast<uint4*>(a.pq + prow) = pack8_t<T>(mo);
#pragma unroll
        for (int e = 0; e < 8; ++e) mo[e] = acck[l][e] * inv_c;
        *reinterpret_cast<uint4*>(a.pk + prow) = pack8_t<T>(mo);
#pragma unroll
        for (int e = 0; e < 8; ++e) mo[e] = accv[l][e] * inv_c;
        *reinterpret_cast<uint4*>(a.pv + prow) = pack8_t<T>(mo);
        if (l16 == 0) {
          a.sqk[srow + a.off[lvl] + node] = mq[l];
          a.skq[srow + a.off[lvl] + node] = mk[l];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) { accq[l][e] = 0.f; acck[l][e] = 0.f; accv[l][e] = 0.f; }
        mq[l] = -INFINITY; mk[l] = -INFINITY;
      }
    }
  };
  // Tokens in chunks of PYR_CHUNK with every load of a chunk issued before the
  // first is used, so a wave keeps PYR_CHUNK rows per tensor in flight instead
  // of one; tokens are still summed in order.
  int t = t0;
  for (; t + PYR_CHUNK <= t1; t += PYR_CHUNK) {
    uint4 cq[PYR_CHUNK], ck[PYR_CHUNK], cv[PYR_CHUNK];
    float gq[PYR_CHUNK], gk[PYR_CHUNK];
#pragma unroll
    for (int i = 0; i < PYR_CHUNK; ++i) {
      const int64_t o = xoff + (int64_t)(t + i) * a.ss;
      cq[i] = ld16(a.xq + o);
      ck[i] = ld16(a.xk + o);
      cv[i] = ld16(a.xv + o);
      gq[i] = GIVEN ? a.sqk[srow + t + i] : 0.f;
      gk[i] = GIVEN ? a.skq[srow + t + i] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < PYR_CHUNK; ++i) token(t + i, cq[i], ck[i], cv[i], gq[i], gk[i]);
  }
  for (; t < t1; ++t) {
    const int64_t o = xoff + (int64_t)t * a.ss;
    token(t, ld16(a.xq + o), ld16(a.xk + o), ld16(a.xv + o), GIVEN ? a.sqk[srow + t] : 0.f,
          GIVEN ? a.skq[srow + t] : 0.f);
  }
}

struct PyrBwdArgs {
  const bf16_t *gq, *gk, *gv;
  int64_t gb, gh, gs;
  const int32_t* inv;
  bf16_t *dq, *dk, *dv;
  int64_t ob, os, oh;  // strides of the three outputs (element units)
  const float* fs;     // ROPE: (cos, sin) table; dq, dk are rotated back by -theta
  int B, S, H, L, shift, S_tot;
  int off[9], len[9];
  long long rows;
  int chunks;  // 16-token chunks per (b, h)
};

// One 16-lane group per (b, t, h) row, 8 d each; a block covers 16 consecutive
// tokens of one (b, h), so the rows of a pooled node spanning up to 16 tokens
// are read by one block (the wave or block coalesces the repeats instead of
// several blocks fetching the row through L2), and runs of 32 consecutive
// chunks of a head stay on one XCD (`xcd_run`; one whole head per XCD left the
// XCDs unevenly loaded, as the gathered rows per token differ by head).  All
// levels' inverse lookups
// are issued first, then all gradient-row loads, so a row costs two dependent
// memory round trips instead of two per level.  ROPE: the q and k sums are
// the gradients of rotated rows; they are rotated back (the adjoint of the
// forward rotation) in fp32 before the one rounding.
template <typename T, int NL, bool ROPE>
__global__ __launch_bounds__(256) void pyramid_bwd_kernel(const PyrBwdArgs a) {
  const int tid = threadIdx.x;
  const long long blk = xcd_run(blockIdx.x, gridDim.x, 32);
  const long long bh = blk / a.chunks;
  const int t = (int)(blk - bh * a.chunks) * 16 + (tid >> 4);
  const int l16 = tid & 15;
  if (t >= a.S) return;
  const int h = (int)(bh % a.H);
  const int b = (int)(bh / a.H);
  const size_t irow = (size_t)(b * a.H + h) * a.S_tot;
  const int64_t gbase = (int64_t)b * a.gb + (int64_t)h * a.gh + 8 * l16;
  int s[NL];
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const int node = t >> (l * a.shift);
    const int r = a.off[l + 1] + node;
    s[l] = node < a.len[l + 1] ? (a.inv ? a.inv[irow + r] : r) : -1;
  }
  const uint4 z = make_uint4(0, 0, 0, 0);
  uint4 gq[NL], gk[NL], gv[NL];
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const int64_t go = gbase + (int64_t)max(s[l], 0) * a.gs;
    gq[l] = (a.gq && s[l] >= 0) ? ld16(a.gq + go) : z;
    gk[l] = (a.gk && s[l] >= 0) ? ld16(a.gk + go) : z;
    gv[l] = (a.gv && s[l] >= 0) ? ld16(a.gv + go) : z;
  }
  float fq[8] = {0}, fk[8] = {0}, fv[8] = {0};
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const float w = 1.0f / (float)(1 << (l * a.shift));
    float g[8];
    unpack8_t<T>(gq[l], g);
#pragma unroll
    for (int e = 0; e < 8; ++e) fq[e] = fmaf(g[e], w, fq[e]);
    unpack8_t<T>(gk[l], g);
#pragma unroll
    for (int e = 0; e < 8; ++e) fk[e] = fmaf(g[e], w, fk[e]);
    unpack8_t<T>(gv[l], g);
#pragma unroll
    for (int e = 0; e < 8; ++e) fv[e] = fmaf(g[e], w, fv[e]);
  }
  if (ROPE) {
    float4 c01, c23;
    rope_freqs8(a.fs, t, LH_D, 8 * l16, c01, c23);
    rope_rotate8<false>(fq, c01, c23);
    rope_rotate8<false>(fk, c01, c23);
  }
  const int64_t o = (int64_t)b * a.ob + (int64_t)t * a.os + (int64_t)h * a.oh + 8 * l16;
  if (a.dq) store16_nt(a.dq + o, pack8_t<T>(fq));
  if (a.dk) store16_nt(a.dk + o, pack8_t<T>(fk));
  if (a.dv) store16_nt(a.dv + o, pack8_t<T>(fv));
}

template <typename T, int NL>
int launch_fwd(const PyrArgs& a, bool given, hipStream_t st) {
  const int blocks = (a.units + 15) / 16;
  if (a.fs)
    hipLaunchKernelGGL((pyramid_fwd_kernel<BF16, NL, false, true>), dim3(blocks), dim3(256), 0, st, a);
  else if (given)
    hipLaunchKernelGGL((pyramid_fwd_kernel<T, NL, true, false>), dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((pyramid_fwd_kernel<T, NL, false, false>), dim3(blocks), dim3(256), 0, st, a);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

namespace {

int pyramid_fwd_impl(const void* xq, const void* xk, const void* xv, int64_t sb, int64_t ss, int64_t sh,
                     const float* freqs, void* rq, void* rk, int64_t rb, int64_t rs, int64_t rh,
                     void* pq, void* pk, void* pv, int64_t pb, int64_t ps, int64_t ph,
                     float* scores_qk, float* scores_kq, int B, int S, int H, int D, int L, int p,
                     bool given, int dtype, void* stream) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!valid_dtype(dtype) || (freqs && dtype != LH_DTYPE_BF16)) return LH_ERR_INVALID_ARG;
  if (!xq || !xk || !xv || !scores_qk || !scores_kq || B <= 0 || H <= 0 || S <= 0) return LH_ERR_INVALID_ARG;
  const int shift = ilog2_exact(p);
  if (shift <= 0 || L < 1) return LH_ERR_INVALID_ARG;
  if (L > 6) return LH_ERR_UNSUPPORTED;
  if (L > 1 && (!pq || !pk || !pv)) return LH_ERR_INVALID_ARG;
  if ((sb | ss | sh) % 8 || (L > 1 && (pb | ps | ph) % 8)) return LH_ERR_INVALID_ARG;
  if (!aligned16(xq) || !aligned16(xk) || !aligned16(xv) || (L > 1 && (!aligned16(pq) || !aligned16(pk) || !aligned16(pv))))
    return LH_ERR_INVALID_ARG;
  if (freqs && (!rq || !rk || !aligned16(freqs) || !aligned16(rq) || !aligned16(rk) || (rb | rs | rh) % 8))
    return LH_ERR_INVALID_ARG;
  Pyramid g;
  if (!make_pyramid(S, L, p, &g)) return LH_ERR_INVALID_ARG;
  PyrArgs a{};
  a.xq = (const bf16_t*)xq; a.xk = (const bf16_t*)xk; a.xv = (const bf16_t*)xv;
  a.sb = sb; a.ss = ss; a.sh = sh;
  a.pq = (bf16_t*)pq; a.pk = (bf16_t*)pk; a.pv = (bf16_t*)pv;
  a.pb = pb; a.ps = ps; a.ph = ph;
  a.sqk = scores_qk; a.skq = scores_kq;
  a.fs = freqs; a.rq = (bf16_t*)rq; a.rk = (bf16_t*)rk;
  a.rb = rb; a.rs = rs; a.rh = rh;
  a.B = B; a.S = S; a.H = H; a.L = L; a.shift = shift; a.S_tot = g.total;
  a.cmax = ipow(p, L - 1);
  if (a.cmax > 4096) return LH_ERR_UNSUPPORTED;
  a.nspan = (S + a.cmax - 1) / a.cmax;
  const long long units = (long long)B * a.nspan * H;
  if (units > (1LL << 30)) return LH_ERR_UNSUPPORTED;
  a.units = (int)units;
  for (int l = 1; l <= L; ++l) { a.off[l] = g.off[l]; a.len[l] = g.len[l]; }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc = LH_OK;
  LH_DISPATCH_DTYPE(dtype, switch (L - 1) {
    case 0: rc = launch_fwd<T, 0>(a, given, st); break;
    case 1: rc = launch_fwd<T, 1>(a, given, st); break;
    case 2: rc = launch_fwd<T, 2>(a, given, st); break;
    case 3: rc = launch_fwd<T, 3>(a, given, st); break;
    case 4: rc = launch_fwd<T, 4>(a, given, st); break;
    default: rc = launch_fwd<T, 5>(a, given, st); break;
  });
  return rc;
}

template <typename T, bool ROPE>
void launch_bwd(const PyrBwdArgs& a, dim3 grid, hipStream_t st) {
  const dim3 blk(256);
  switch (a.L) {
    case 1: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 1, ROPE>), grid, blk, 0, st, a); break;
    case 2: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 2, ROPE>), grid, blk, 0, st, a); break;
    case 3: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 3, ROPE>), grid, blk, 0, st, a); break;
    case 4: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 4, ROPE>), grid, blk, 0, st, a); break;
    case 5: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 5, ROPE>), grid, blk, 0, st, a); break;
    case 6: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 6, ROPE>), grid, blk, 0, st, a); break;
    case 7: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 7, ROPE>), grid, blk, 0, st, a); break;
    default: hipLaunchKernelGGL((pyramid_bwd_kernel<T, 8, ROPE>), grid, blk, 0, st, a); break;
  }
}

int pyramid_bwd_impl(const void* gq, const void* gk, const void* gv, int64_t gb, int64_t gh, int64_t gs,
                     const int32_t* inverse, const float* freqs, void* dxq, void* dxk, void* dxv, int64_t ob,
                     int64_t os, int64_t oh, int B, int S, int H, int D, int L, int p, int dtype, void* stream) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (B <= 0 || H <= 0 || S <= 0 || L < 1 || L > 8) return LH_ERR_INVALID_ARG;
  if (!valid_dtype(dtype) || (freqs && dtype != LH_DTYPE_BF16)) return LH_ERR_INVALID_ARG;
  const int shift = ilog2_exact(p);
  if (shift <= 0) return LH_ERR_INVALID_ARG;
  if ((gq != nullptr) != (dxq != nullptr) || (gk != nullptr) != (dxk != nullptr) || (gv != nullptr) != (dxv != nullptr))
    return LH_ERR_INVALID_ARG;
  if ((gb | gh | gs) % 8 || (ob | os | oh) % 8) return LH_ERR_INVALID_ARG;
  for (const void* x : {gq, gk, gv, (const void*)dxq, (const void*)dxk, (const void*)dxv})
    if (x && !aligned16(x)) return LH_ERR_INVALID_ARG;
  if (freqs && !aligned16(freqs)) return LH_ERR_INVALID_ARG;
  Pyramid g;
  if (!make_pyramid(S, L, p, &g)) return LH_ERR_INVALID_ARG;
  PyrBwdArgs a{};
  a.gq = (const bf16_t*)gq; a.gk = (const bf16_t*)gk; a.gv = (const bf16_t*)gv;
  a.gb = gb; a.gh = gh; a.gs = gs; a.inv = inverse;
  a.dq = (bf16_t*)dxq; a.dk = (bf16_t*)dxk; a.dv = (bf16_t*)dxv;
  a.ob = ob; a.os = os; a.oh = oh; a.fs = freqs;
  a.B = B; a.S = S; a.H = H; a.L = L; a.shift = shift; a.S_tot = g.total;
  for (int l = 1; l <= L; ++l) { a.off[l] = g.off[l]; a.len[l] = g.len[l]; }
  a.rows = (long long)B * S * H;
  a.chunks = (S + 15) / 16;
  const long long blocks = (long long)B * H * a.chunks;
  if (blocks > 2147483647LL) return LH_ERR_UNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (freqs)
    launch_bwd<BF16, true>(a, dim3((unsigned)blocks), st);
  else
    LH_DISPATCH_DTYPE(dtype, launch_bwd<T, false>(a, dim3((unsigned)blocks), st));
  LH_CHECK_LAUNCH();
  return LH_OK;
}

}  // namespace

extern "C" int lh_pyramid_fwd(const void* xq, const void* xk, const void* xv, int64_t sb, int64_t ss, int64_t sh,
                              void* pq, void* pk, void* pv, int64_t pb, int64_t ps, int64_t ph,
                              float* scores_qk, float* scores_kq, int B, int S, int H, int D, int L, int p,
                              int base_scores_given, int dtype, void* stream) {
  return pyramid_fwd_impl(xq, xk, xv, sb, ss, sh, nullptr, nullptr, nullptr, 0, 0, 0, pq, pk, pv, pb, ps, ph,
                          scores_qk, scores_kq, B, S, H, D, L, p, base_scores_given != 0, dtype, stream);
}

extern "C" int lh_rope_pyramid_fwd(const void* xq, const void* xk, const void* xv, int64_t sb, int64_t ss,
                                   int64_t sh, const float* freqs, void* rq, void* rk, int64_t rb, int64_t rs,
                                   int64_t rh, void* pq, void* pk, void* pv, int64_t pb, int64_t ps, int64_t ph,
                                   float* scores_qk, float* scores_kq, int B, int S, int H, int D, int L, int p,
                                   void* stream) {
  if (!freqs) return LH_ERR_INVALID_ARG;
  return pyramid_fwd_impl(xq, xk, xv, sb, ss, sh, freqs, rq, rk, rb, rs, rh, pq, pk, pv, pb, ps, ph, scores_qk,
                          scores_kq, B, S, H, D, L, p, false, LH_DTYPE_BF16, stream);
}

extern "C" int lh_pyramid_bwd(const void* gq, const void* gk, const void* gv, int64_t gb, int64_t gh, int64_t gs,
                              const int32_t* inverse, void* dxq, void* dxk, void* dxv, int B, int S, int H, int D,
                              int L, int p, int dtype, void* stream) {
  const int64_t oh = D, os = (int64_t)H * D, ob = (int64_t)S * os;
  return pyramid_bwd_impl(gq, gk, gv, gb, gh, gs, inverse, nullptr, dxq, dxk, dxv, ob, os, oh, B, S, H, D, L, p,
                          dtype, stream);
}

extern "C" int lh_pyramid_rope_bwd(const void* gq, const void* gk, const void* gv, int64_t gb, int64_t gh,
                                   int64_t gs, const int32_t* inverse, const float* freqs, void* dxq, void* dxk,
                                   void* dxv, int64_t ob, int64_t os, int64_t oh, int B, int S, int H, int D, int L,
                                   int p, void* stream) {
  if (!freqs) return LH_ERR_INVALID_ARG;
  return pyramid_bwd_impl(gq, gk, gv, gb, gh, gs, inverse, freqs, dxq, dxk, dxv, ob, os, oh, B, S, H, D, L, p,
                          LH_DTYPE_BF16, stream);
}

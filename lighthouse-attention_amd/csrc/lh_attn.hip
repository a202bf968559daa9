// Causal attention over gathered rows on gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Replaces the three torch.gather calls and the inner causal SDPA of
// LighthouseLocal.forward (src/lighthouse_selection.py:800-815) and, with an
// identity row map and a norm epilogue, the two SDPA calls of
// DilatedLighthouseScorer.forward (:642-653).
//
// Layout choices (one 64-lane wave computes 32 queries x 64 keys per step;
// 8 waves share each K/V tile in the query-stationary kernels):
//   * Scores are formed transposed, S^T = K Q^T, so an MFMA output column is a
//     query: lane l holds query l%32 and 16 keys per 32x32 block.  Row max and
//     row sum of the online softmax are in-lane plus one exchange with lane
//     l^32, and the per-query rescale of O is a per-lane scalar.
//   * The exp'd scores feed P V directly from registers: the C-layout of S^T
//     (key = 8*(v/4) + 4*(l/32) + v%4) is used as the k-order of the next MFMA,
//     and the A operand V^T is read from the row-major V tile with the
//     transposing LDS read ds_read_b64_tr_b16 in the same key order.
//   * LDS tiles are row-major, unpadded and XOR-swizzled per 16-byte chunk, and
//     are filled by direct global->LDS loads (global_load_lds_dwordx4): no
//     register staging, no transposed copies.  Two buffers per operand; the
//     next tile's loads are issued before the current tile's MFMAs.
//   * Rows are gathered on the fly: row s of (b, h) is read through
//     indices[b, h, s] from the base [B, S, H, D] tensor or the pooled
//     [B, Sp, H, D] tensor (32-bit element offsets within one (b, h); K and V
//     share them).  Rows past the end are clamped to the last row and masked,
//     so loads never branch.
//   * One tile body serves masked and unmasked tiles (a wave-uniform flag
//     guards the mask code), so accumulators keep one register assignment.
//   * The running maximum is only raised when a row's maximum grows by more
//     than 2^8 (in exp2 units); until then exp'd scores may reach 2^8, which
//     bf16 and fp32 hold exactly as well as values <= 1, and the O rescale is
//     skipped.
//   * Backward is deterministic: dK/dV in a key-stationary kernel, dQ in a
//     query-stationary kernel, no atomics.
// Softmax runs in the exp2 domain with scale*log2(e); the stored LSE is
// m + log2(l) in that domain.
#include "lh_common.h"

namespace {

constexpr int BMK = 128;  // keys per workgroup of the key-stationary kernel: 4 waves x 32
constexpr int QW = 8;     // waves per workgroup of the query-stationary kernels (32 queries each)
constexpr int BN = 64;   // rows per LDS tile
constexpr float RESCALE_LOG2 = 8.0f;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

struct Rows {
  const bf16_t *q, *k, *v, *qp, *kp, *vp;
  int64_t sb, ss, sh, pb, ps, ph;
  int split;
  const int32_t* idx;  // [BH, n] or null (identity)
};

struct AttnArgs {
  Rows R;
  int B, H, n, nq, BH;
  float sl2;    // softmax scale * log2(e)
  float scale;  // softmax scale
  bf16_t* out;  // fwd: O [BH, n, D]
  float* lse;   // fwd: [BH, n]
  // norm epilogue (dilated scorer): token t = s*dil + vh/Ho, head vh % Ho
  float* scores;
  int Ho, dil, S_tot;
  // backward
  const bf16_t* dout;
  const float* lse_in;
  const float* delta;
  bf16_t *dq, *dk, *dv;
};

// Row source of one (b, h): uniform base pointers and 32-bit strides.
struct BhRows {
  const bf16_t *q, *k, *v, *qp, *kp, *vp;
  const int32_t* idx;
  int ss, ps, split, last;
};

__device__ __forceinline__ BhRows bh_rows(const AttnArgs& a, int bh) {
  const Rows& R = a.R;
  const int b = bh / a.H, h = bh % a.H;
  BhRows m;
  const int64_t ob = (int64_t)b * R.sb + (int64_t)h * R.sh;
  const int64_t op = (int64_t)b * R.pb + (int64_t)h * R.ph;
  m.q = R.q + ob; m.k = R.k + ob; m.v = R.v + ob;
  m.qp = R.qp + op; m.kp = R.kp + op; m.vp = R.vp + op;
  m.idx = R.idx ? R.idx + (int64_t)bh * a.n : nullptr;
  m.ss = (int)R.ss; m.ps = (int)R.ps; m.split = R.split; m.last = a.n - 1;
  return m;
}

// element offset of selected row s (clamped to the last row); `pooled` picks the tensor
__device__ __forceinline__ uint32_t row_off(const BhRows& m, int s, bool& pooled) {
  s = min(s, m.last);
  const int r = m.idx ? m.idx[s] : s;
  pooled = r >= m.split;
  return pooled ? (uint32_t)(r - m.split) * (uint32_t)m.ps : (uint32_t)r * (uint32_t)m.ss;
}

__device__ __forceinline__ floatx16 mfma(const u32x4 a, const u32x4 b, const floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

__device__ __forceinline__ uint32_t cvt2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ u32x4 ldg16(const bf16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Blocks are dispatched round-robin over the 8 XCDs; give each XCD a
// contiguous run of (b, h) so K/V rows stay in that XCD's L2, and run the
// heaviest causal blocks first.
__device__ __forceinline__ void schedule(int w, int nblk, int BH, int& bh, int& blk, bool heavy_last) {
  const int total = nblk * BH;
  int t = w;
  if ((total & 7) == 0) t = (w & 7) * (total >> 3) + (w >> 3);
  bh = t / nblk;
  const int r = t % nblk;
  blk = heavy_last ? (nblk - 1 - r) : r;
}

// ---------------------------------------------------------------------------
// LDS tiles: 64 rows x 128 bf16, rows unpadded (256 B), 16-byte chunks
// swizzled as chunk ^ swz(row).  swz is a bijection on every 16 consecutive
// rows (so 128-bit row reads of 16 rows at one chunk hit distinct banks) and
// gives 4 consecutive rows distinct high bits (so the transposing reads of a
// 4-row x 4-chunk block hit distinct banks).  Tiles are filled by direct
// global->LDS loads: lane l of a 16-byte load writes LDS base + 16*l, so each
// lane fetches the logical chunk that the swizzle puts in its slot.
// ---------------------------------------------------------------------------
constexpr int TILE = BN * LH_D;  // elements per tile (16 KB)

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ u32x2 ld_tr16(const bf16_t* p) {
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p));
  return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ void g2l16(const bf16_t* g, bf16_t* lds_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_base, 16, 0, 0);
}

// Wave w fills rows 16w .. 16w+15 of a 64-row tile with four 1 KB direct loads
// of 4 rows each.  The selected-row indices of those rows are loaded one tile
// ahead (load_rows) so issuing a tile never waits on an index load.
template <int NW>
__device__ __forceinline__ void load_rows(int (&r)[16 / NW], const BhRows& m, int row0, int w, int lane) {
#pragma unroll
  for (int i = 0; i < 16 / NW; ++i) {
    const int s = min(row0 + (64 / NW) * w + 4 * i + (lane >> 4), m.last);
    r[i] = m.idx ? m.idx[s] : s;
  }
}

// (tile2 != null: a second tensor with the same row map, e.g. V beside K)
template <int NW>
__device__ __forceinline__ void issue_rows(bf16_t* tile, const bf16_t* base, const bf16_t* pool, bf16_t* tile2,
                                           const bf16_t* base2, const bf16_t* pool2, const BhRows& m,
                                           const int (&rr)[16 / NW], int w, int lane) {
  const int rsub = lane >> 4, slot = lane & 15;
#pragma unroll
  for (int i = 0; i < 16 / NW; ++i) {
    const int r = (64 / NW) * w + 4 * i + rsub;
    const bool pooled = rr[i] >= m.split;
    const uint32_t o = (pooled ? (uint32_t)(rr[i] - m.split) * (uint32_t)m.ps : (uint32_t)rr[i] * (uint32_t)m.ss) +
                       8 * (slot ^ swz(r));
    g2l16((pooled ? pool : base) + o, tile + ((64 / NW) * w + 4 * i) * LH_D);
    if (tile2) g2l16((pooled ? pool2 : base2) + o, tile2 + ((64 / NW) * w + 4 * i) * LH_D);
  }
}

template <int NW>
__device__ __forceinline__ void issue_dense(bf16_t* tile, const bf16_t* base, int last, int row0, int w, int lane) {
  const int rsub = lane >> 4, slot = lane & 15;
#pragma unroll
  for (int i = 0; i < 16 / NW; ++i) {
    const int r = (64 / NW) * w + 4 * i + rsub;
    g2l16(base + (uint32_t)min(row0 + r, last) * LH_D + 8 * (slot ^ swz(r)), tile + ((64 / NW) * w + 4 * i) * LH_D);
  }
}

// every direct load of this wave has landed in LDS
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0); }

// A operand from tile row r: d = 16c + 8hh .. 16c + 8hh + 7
__device__ __forceinline__ u32x4 op_row(const bf16_t* tile, int r, int c, int hh) {
  return *reinterpret_cast<const u32x4*>(tile + r * LH_D + (((2 * c + hh) ^ swz(r)) << 3));
}

// A operand of X^T: column d = 32db + lane%32; k-slots u are rows
// r0 + 8(u/4) + 4(lane/32) + u%4 (r0 a multiple of 16).  Within each 16-lane
// group, ds_read_b64_tr_b16 returns to lane i, element e, the 16-bit word i%4 of
// the 8 bytes addressed by lane i/4 + 4e; each lane therefore addresses 4
// columns of one row of a 4-row x 16-column block.
__device__ __forceinline__ u32x4 op_tr(const bf16_t* tile, int r0, int db, int lane) {
  const int g = lane >> 4, j = lane & 15;
  const int r = r0 + 4 * (lane >> 5) + (j >> 2);
  const int ch = 4 * db + 2 * (g & 1) + ((j & 3) >> 1);
  const int sub = (j & 1) << 2;
  const u32x2 lo = ld_tr16(tile + r * LH_D + ((ch ^ swz(r)) << 3) + sub);
  const u32x2 hi = ld_tr16(tile + (r + 8) * LH_D + ((ch ^ swz(r + 8)) << 3) + sub);
  return u32x4{lo.x, lo.y, hi.x, hi.y};
}

// 8 fp32 accumulator values v = 8*c2 .. 8*c2+7 -> bf16 B operand
__device__ __forceinline__ u32x4 pack_frag(const floatx16& s, int c2) {
  const int v = 8 * c2;
  return u32x4{cvt2(s[v + 0], s[v + 1]), cvt2(s[v + 2], s[v + 3]), cvt2(s[v + 4], s[v + 5]), cvt2(s[v + 6], s[v + 7])};
}

// key index held in accumulator slot v of a 32-key block
__device__ __forceinline__ int slot_key(int v, int hh) { return 8 * (v >> 2) + 4 * hh + (v & 3); }

__device__ __forceinline__ void store_rows_bf16(bf16_t* row, const floatx16 (&acc)[4], float sc, int hh) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w.x = cvt2(acc[d][4 * g + 0] * sc, acc[d][4 * g + 1] * sc);
      w.y = cvt2(acc[d][4 * g + 2] * sc, acc[d][4 * g + 3] * sc);
      *reinterpret_cast<u32x2*>(row + d * 32 + 8 * g + 4 * hh) = w;
    }
  }
}

// ===========================================================================
// forward (query-stationary)
// ===========================================================================
struct FwdState {
  floatx16 o[4];
  float m;  // running max in raw (unscaled) score units
  float l;  // this lane's half of the row sum
};

__device__ __forceinline__ void fwd_tile(FwdState& st, const u32x4 (&qf)[8], const bf16_t* Ks, const bf16_t* Vs,
                                         int k0, int my_q, int n, int lane, float sl2, bool mask) {
  const int l32 = lane & 31, hh = lane >> 5;
  floatx16 s[2];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    s[kb] = mfma(op_row(Ks, kb * 32 + l32, 0, hh), qf[0], floatx16{});
#pragma unroll
    for (int c = 1; c < 8; ++c) s[kb] = mfma(op_row(Ks, kb * 32 + l32, c, hh), qf[c], s[kb]);
  }
  __builtin_amdgcn_s_setprio(0);
  if (mask) {  // wave-uniform: only tiles that cross the diagonal or the end
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = k0 + kb * 32 + slot_key(v, hh);
        if (key > my_q || key >= n) s[kb][v] = -INFINITY;
      }
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kb][v]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const bool raise = mx > st.m + RESCALE_LOG2 / sl2;
  if (__any(raise)) {
    const float m_new = raise ? mx : st.m;
    const float alpha = raise ? ex2((st.m - m_new) * sl2) : 1.f;  // 0 on the first raise (m = -inf)
    st.l *= alpha;
#pragma unroll
    for (int d = 0; d < 4; ++d) st.o[d] *= alpha;
    st.m = m_new;
  }
  const float nm = (st.m == -INFINITY) ? 0.f : -st.m * sl2;
  float ls = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float p = ex2(fmaf(s[kb][v], sl2, nm));
      s[kb][v] = p;
      ls += p;
    }
  }
  st.l += ls;
  u32x4 pf[2][2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    pf[kb][0] = pack_frag(s[kb], 0);
    pf[kb][1] = pack_frag(s[kb], 1);
  }
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) st.o[d] = mfma(op_tr(Vs, kb * 32 + 16 * c2, d, lane), pf[kb][c2], st.o[d]);
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

template <int EPI>  // 0: O + LSE;  1: bf16-rounded row norms of O into `scores`
__global__ __launch_bounds__(64 * QW, 8 / QW) void attn_fwd_kernel(const AttnArgs a) {
  constexpr int BM = 32 * QW;
  __shared__ __attribute__((aligned(1024))) bf16_t K0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t K1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V1[TILE];
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int bh, qb;
  schedule(blockIdx.x, a.nq, a.BH, bh, qb, true);
  const int n = a.n;
  const BhRows m = bh_rows(a, bh);
  const int q0 = qb * BM, qw = q0 + wave * 32, my_q = qw + l32;

  u32x4 qf[8];
  {
    bool pooled;
    const uint32_t o = row_off(m, my_q, pooled) + 8 * hh;
    const bf16_t* p = (pooled ? m.qp : m.q) + o;
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = ldg16(p + 16 * c);
  }

  const int kend = min(q0 + BM, n);
  const int nt = (kend + BN - 1) / BN;
  int rr[16 / QW];
  load_rows<QW>(rr, m, 0, wave, lane);
  issue_rows<QW>(K0, m.k, m.kp, V0, m.v, m.vp, m, rr, wave, lane);
  load_rows<QW>(rr, m, BN, wave, lane);
  wait_loads();
  __syncthreads();

  FwdState st;
#pragma unroll
  for (int d = 0; d < 4; ++d) st.o[d] = floatx16{};
  st.m = -INFINITY;
  st.l = 0.f;
  // tiles whose 64 keys are all <= this wave's first query and < n need no mask
  const int nfull = min((qw + 1) / BN, n / BN);

  auto step = [&](int j, const bf16_t* Ks, const bf16_t* Vs, bf16_t* Kn, bf16_t* Vn) {
    const int k0 = j * BN;
    if (j + 1 < nt) issue_rows<QW>(Kn, m.k, m.kp, Vn, m.v, m.vp, m, rr, wave, lane);
    if (j + 2 < nt) load_rows<QW>(rr, m, k0 + 2 * BN, wave, lane);
    if (j < nt && k0 <= qw + 31) fwd_tile(st, qf, Ks, Vs, k0, my_q, n, lane, a.sl2, j >= nfull);
    wait_loads();
    __syncthreads();
  };
  for (int j = 0; j < nt; j += 2) {
    step(j, K0, V0, K1, V1);
    step(j + 1, K1, V1, K0, V0);
  }

  if (my_q >= n) return;
  const float l = st.l + __shfl_xor(st.l, 32);
  const float inv_l = l > 0.f ? 1.0f / l : 0.f;
  if (EPI == 0) {
    store_rows_bf16(a.out + ((int64_t)bh * n + my_q) * LH_D, st.o, inv_l, hh);
    if (hh == 0) a.lse[(int64_t)bh * n + my_q] = l > 0.f ? st.m * a.sl2 + __log2f(l) : -INFINITY;
  } else {
    float ss = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const uint32_t w = cvt2(st.o[d][v] * inv_l, st.o[d][v + 1] * inv_l);
        const float x0 = __uint_as_float(w << 16), x1 = __uint_as_float(w & 0xffff0000u);
        ss = fmaf(x0, x0, ss);
        ss = fmaf(x1, x1, ss);
      }
    }
    ss += __shfl_xor(ss, 32);
    if (hh == 0) {
      const int vh = bh % a.H;  // virtual head of the dilated view
      const int b = bh / a.H;
      const int t = my_q * a.dil + vh / a.Ho;
      const int ho = vh % a.Ho;
      a.scores[((int64_t)b * a.Ho + ho) * a.S_tot + t] = __uint_as_float(cvt2(sqrtf(ss), 0.f) << 16);
    }
  }
}

// ===========================================================================
// backward dQ (query-stationary)
// ===========================================================================
__device__ __forceinline__ void dq_tile(floatx16 (&acc)[4], const u32x4 (&qf)[8], const u32x4 (&df)[8],
                                        const bf16_t* Ks, const bf16_t* Vs, int k0, int my_q, int n, int lane,
                                        float sl2, float nlse, float dlt, bool mask) {
  const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    __builtin_amdgcn_s_setprio(1);
    floatx16 s = mfma(op_row(Ks, kb * 32 + l32, 0, hh), qf[0], floatx16{});
    floatx16 dp = mfma(op_row(Vs, kb * 32 + l32, 0, hh), df[0], floatx16{});
#pragma unroll
    for (int c = 1; c < 8; ++c) {
      s = mfma(op_row(Ks, kb * 32 + l32, c, hh), qf[c], s);
      dp = mfma(op_row(Vs, kb * 32 + l32, c, hh), df[c], dp);
    }
    __builtin_amdgcn_s_setprio(0);
    if (mask) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = k0 + kb * 32 + slot_key(v, hh);
        if (key > my_q || key >= n) s[v] = -INFINITY;
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) s[v] = ex2(fmaf(s[v], sl2, nlse)) * (dp[v] - dlt);
    const u32x4 f0 = pack_frag(s, 0), f1 = pack_frag(s, 1);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      acc[d] = mfma(op_tr(Ks, kb * 32, d, lane), f0, acc[d]);
      acc[d] = mfma(op_tr(Ks, kb * 32 + 16, d, lane), f1, acc[d]);
    }
    __builtin_amdgcn_s_setprio(0);
  }
}

__global__ __launch_bounds__(64 * QW, 8 / QW) void attn_bwd_dq_kernel(const AttnArgs a) {
  constexpr int BM = 32 * QW;
  __shared__ __attribute__((aligned(1024))) bf16_t K0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t K1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V1[TILE];
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int bh, qb;
  schedule(blockIdx.x, a.nq, a.BH, bh, qb, true);
  const int n = a.n;
  const BhRows m = bh_rows(a, bh);
  const int q0 = qb * BM, qw = q0 + wave * 32, my_q = qw + l32;
  const int qc = min(my_q, n - 1);

  u32x4 qf[8], df[8];
  {
    bool pooled;
    const uint32_t o = row_off(m, my_q, pooled) + 8 * hh;
    const bf16_t* p = (pooled ? m.qp : m.q) + o;
    const bf16_t* pd = a.dout + ((int64_t)bh * n + qc) * LH_D + 8 * hh;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      qf[c] = ldg16(p + 16 * c);
      df[c] = ldg16(pd + 16 * c);
    }
  }
  const float nlse = -a.lse_in[(int64_t)bh * n + qc];
  const float dlt = a.delta[(int64_t)bh * n + qc];

  const int kend = min(q0 + BM, n);
  const int nt = (kend + BN - 1) / BN;
  int rr[16 / QW];
  load_rows<QW>(rr, m, 0, wave, lane);
  issue_rows<QW>(K0, m.k, m.kp, V0, m.v, m.vp, m, rr, wave, lane);
  load_rows<QW>(rr, m, BN, wave, lane);
  wait_loads();
  __syncthreads();

  floatx16 acc[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) acc[d] = floatx16{};
  const int nfull = min((qw + 1) / BN, n / BN);

  auto step = [&](int j, const bf16_t* Ks, const bf16_t* Vs, bf16_t* Kn, bf16_t* Vn) {
    const int k0 = j * BN;
    if (j + 1 < nt) issue_rows<QW>(Kn, m.k, m.kp, Vn, m.v, m.vp, m, rr, wave, lane);
    if (j + 2 < nt) load_rows<QW>(rr, m, k0 + 2 * BN, wave, lane);
    if (j < nt && k0 <= qw + 31) dq_tile(acc, qf, df, Ks, Vs, k0, my_q, n, lane, a.sl2, nlse, dlt, j >= nfull);
    wait_loads();
    __syncthreads();
  };
  for (int j = 0; j < nt; j += 2) {
    step(j, K0, V0, K1, V1);
    step(j + 1, K1, V1, K0, V0);
  }

  if (my_q >= n) return;
  store_rows_bf16(a.dq + ((int64_t)bh * n + my_q) * LH_D, acc, a.scale, hh);
}

// ===========================================================================
// backward dK, dV (key-stationary)
// ===========================================================================
__device__ __forceinline__ void dkdv_tile(floatx16 (&dka)[4], floatx16 (&dva)[4], const u32x4 (&kf)[8],
                                          const u32x4 (&vf)[8], const bf16_t* Qs, const bf16_t* Ds, const float* Ls,
                                          const float* Dl, int q0t, int my_k, int n, int lane, float sl2, bool mask) {
  const int l32 = lane & 31, hh = lane >> 5;
  // one 32-query half at a time keeps the live set to one S and one dP block
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    __builtin_amdgcn_s_setprio(1);
    floatx16 s = mfma(op_row(Qs, qb * 32 + l32, 0, hh), kf[0], floatx16{});
    floatx16 dp = mfma(op_row(Ds, qb * 32 + l32, 0, hh), vf[0], floatx16{});
#pragma unroll
    for (int c = 1; c < 8; ++c) {
      s = mfma(op_row(Qs, qb * 32 + l32, c, hh), kf[c], s);
      dp = mfma(op_row(Ds, qb * 32 + l32, c, hh), vf[c], dp);
    }
    __builtin_amdgcn_s_setprio(0);
    if (mask) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int q = q0t + qb * 32 + slot_key(v, hh);
        if (my_k > q || q >= n) s[v] = -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int qi = qb * 32 + 8 * g + 4 * hh;
      const float4 l4 = *reinterpret_cast<const float4*>(Ls + qi);  // holds -lse
      const float4 d4 = *reinterpret_cast<const float4*>(Dl + qi);
      const float nl[4] = {l4.x, l4.y, l4.z, l4.w};
      const float dd[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = 4 * g + e;
        const float p = ex2(fmaf(s[v], sl2, nl[e]));
        s[v] = p;
        dp[v] = p * (dp[v] - dd[e]);
      }
    }
    const u32x4 p0 = pack_frag(s, 0), p1 = pack_frag(s, 1);
    const u32x4 s0 = pack_frag(dp, 0), s1 = pack_frag(dp, 1);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      dva[d] = mfma(op_tr(Ds, qb * 32, d, lane), p0, dva[d]);
      dva[d] = mfma(op_tr(Ds, qb * 32 + 16, d, lane), p1, dva[d]);
      dka[d] = mfma(op_tr(Qs, qb * 32, d, lane), s0, dka[d]);
      dka[d] = mfma(op_tr(Qs, qb * 32 + 16, d, lane), s1, dka[d]);
    }
    __builtin_amdgcn_s_setprio(0);
  }
}

__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(1024))) bf16_t Q0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t Q1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t D0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t D1[TILE];
  __shared__ __attribute__((aligned(16))) float L0[2 * BN];  // -lse then delta
  __shared__ __attribute__((aligned(16))) float L1[2 * BN];
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int bh, kblk;
  schedule(blockIdx.x, a.nq, a.BH, bh, kblk, false);  // early key blocks see the most queries
  const int n = a.n;
  const BhRows m = bh_rows(a, bh);
  const int k0 = kblk * BMK, kw = k0 + wave * 32, my_k = kw + l32;

  u32x4 kf[8], vf[8];
  {
    bool pooled;
    const uint32_t o = row_off(m, my_k, pooled) + 8 * hh;
    const bf16_t* pk = (pooled ? m.kp : m.k) + o;
    const bf16_t* pv = (pooled ? m.vp : m.v) + o;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      kf[c] = ldg16(pk + 16 * c);
      vf[c] = ldg16(pv + 16 * c);
    }
  }

  const int jt0 = k0 / BN;
  const int nt = (n + BN - 1) / BN;
  const bf16_t* dbase = a.dout + (int64_t)bh * n * LH_D;
  const float* lrow = a.lse_in + (int64_t)bh * n;
  const float* drow = a.delta + (int64_t)bh * n;
  // threads 0..63 carry -lse, 64..127 delta of the tile's 64 queries
  auto load_ld = [&](int q0t) -> float {
    if (tid >= 2 * BN) return 0.f;
    const int qq = min(q0t + (tid & (BN - 1)), n - 1);
    return tid < BN ? -lrow[qq] : drow[qq];
  };
  int rr[4];
  load_rows<4>(rr, m, jt0 * BN, wave, lane);
  issue_rows<4>(Q0, m.q, m.qp, nullptr, nullptr, nullptr, m, rr, wave, lane);
  issue_dense<4>(D0, dbase, n - 1, jt0 * BN, wave, lane);
  if (tid < 2 * BN) L0[tid] = load_ld(jt0 * BN);
  load_rows<4>(rr, m, (jt0 + 1) * BN, wave, lane);
  wait_loads();
  __syncthreads();

  floatx16 dka[4], dva[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) { dka[d] = floatx16{}; dva[d] = floatx16{}; }
  // query tiles whose 64 queries are all >= this wave's last key and < n need no mask
  const int jfull = (kw + 31 + BN - 1) / BN;

  auto step = [&](int j, const bf16_t* Qs, const bf16_t* Ds, const float* Ls, bf16_t* Qn, bf16_t* Dn, float* Ln) {
    const int q0t = j * BN;
    float lv = 0.f;
    if (j + 1 < nt) {
      issue_rows<4>(Qn, m.q, m.qp, nullptr, nullptr, nullptr, m, rr, wave, lane);
      issue_dense<4>(Dn, dbase, n - 1, q0t + BN, wave, lane);
      lv = load_ld(q0t + BN);
    }
    if (j + 2 < nt) load_rows<4>(rr, m, q0t + 2 * BN, wave, lane);
    if (j < nt && q0t + BN - 1 >= kw)
      dkdv_tile(dka, dva, kf, vf, Qs, Ds, Ls, Ls + BN, q0t, my_k, n, lane, a.sl2, !(j >= jfull && q0t + BN <= n));
    if (j + 1 < nt && tid < 2 * BN) Ln[tid] = lv;
    wait_loads();
    __syncthreads();
  };
  for (int j = jt0; j < nt; j += 2) {
    step(j, Q0, D0, L0, Q1, D1, L1);
    step(j + 1, Q1, D1, L1, Q0, D0, L0);
  }

  if (my_k >= n) return;
  store_rows_bf16(a.dk + ((int64_t)bh * n + my_k) * LH_D, dka, a.scale, hh);
  store_rows_bf16(a.dv + ((int64_t)bh * n + my_k) * LH_D, dva, 1.0f, hh);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int fill_rows(AttnArgs& a, const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
              const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph, int split,
              const int32_t* indices, int B, int H, int n, int D, float scale) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!q || !k || !v || B <= 0 || H <= 0 || n <= 0) return LH_ERR_INVALID_ARG;
  if (!al16(q) || !al16(k) || !al16(v) || (sb | ss | sh) % 8 || ss <= 0) return LH_ERR_INVALID_ARG;
  const bool need_pool = indices != nullptr;  // pooled rows only reachable through an index map
  if (need_pool && (!qp || !kp || !vp || !al16(qp) || !al16(kp) || !al16(vp) || (pb | ps | ph) % 8 || ps <= 0))
    return LH_ERR_INVALID_ARG;
  if (!(scale > 0.f)) return LH_ERR_INVALID_ARG;
  // Row offsets inside one (b, h) are 32-bit.  Base rows are < split (or < n
  // without an index map); pooled rows r - split are < split too, as every
  // pyramid's pooled levels are shorter than its base level.
  const long long rows = need_pool ? split : n;
  if (rows * ss + LH_D > 0x7fffffffLL || (need_pool && rows * ps + LH_D > 0x7fffffffLL)) return LH_ERR_UNSUPPORTED;
  a.R.q = (const bf16_t*)q; a.R.k = (const bf16_t*)k; a.R.v = (const bf16_t*)v;
  a.R.qp = (const bf16_t*)(qp ? qp : q); a.R.kp = (const bf16_t*)(kp ? kp : k); a.R.vp = (const bf16_t*)(vp ? vp : v);
  a.R.sb = sb; a.R.ss = ss; a.R.sh = sh; a.R.pb = pb; a.R.ps = need_pool ? ps : ss; a.R.ph = ph;
  a.R.split = indices ? split : 0x7fffffff;
  a.R.idx = indices;
  a.B = B; a.H = H; a.n = n; a.BH = B * H;
  a.nq = (n + 32 * QW - 1) / (32 * QW);  // query blocks (the key-stationary launch resets it)
  a.scale = scale;
  a.sl2 = (float)((double)scale * 1.4426950408889634);
  if ((long long)((n + 127) / 128) * a.BH > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
  return LH_OK;
}

}  // namespace

extern "C" int lh_attn_fwd(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                           const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                           int split, const int32_t* indices, int B, int H, int n, int D, float scale, void* out,
                           float* lse, void* stream) {
  AttnArgs a{};
  int rc = fill_rows(a, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale);
  if (rc) return rc;
  if (!out || !lse || !al16(out)) return LH_ERR_INVALID_ARG;
  a.out = (bf16_t*)out; a.lse = lse;
  hipLaunchKernelGGL(attn_fwd_kernel<0>, dim3(a.nq * a.BH), dim3(64 * QW), 0, reinterpret_cast<hipStream_t>(stream),
                     a);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

namespace {
// parts: bit 0 = dK/dV kernel, bit 1 = dQ kernel
int attn_bwd_parts(int parts, const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                   const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph, int split,
                   const int32_t* indices, int B, int H, int n, int D, float scale, const void* dout,
                   const float* lse, const float* delta, void* dq, void* dk, void* dv, void* stream) {
  AttnArgs a{};
  int rc = fill_rows(a, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale);
  if (rc) return rc;
  if (!dout || !lse || !delta || !al16(dout)) return LH_ERR_INVALID_ARG;
  if ((parts & 1) && (!dk || !dv || !al16(dk) || !al16(dv))) return LH_ERR_INVALID_ARG;
  if ((parts & 2) && (!dq || !al16(dq))) return LH_ERR_INVALID_ARG;
  a.dout = (const bf16_t*)dout; a.lse_in = lse; a.delta = delta;
  a.dq = (bf16_t*)dq; a.dk = (bf16_t*)dk; a.dv = (bf16_t*)dv;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (parts & 1) {
    AttnArgs ak = a;
    ak.nq = (a.n + BMK - 1) / BMK;
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel, dim3(ak.nq * ak.BH), dim3(256), 0, st, ak);
    LH_CHECK_LAUNCH();
  }
  if (parts & 2) {
    hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3(a.nq * a.BH), dim3(64 * QW), 0, st, a);
    LH_CHECK_LAUNCH();
  }
  return LH_OK;
}
}  // namespace

extern "C" int lh_attn_bwd(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                           const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                           int split, const int32_t* indices, int B, int H, int n, int D, float scale,
                           const void* dout, const float* lse, const float* delta, void* dq, void* dk, void* dv,
                           void* stream) {
  return attn_bwd_parts(3, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale, dout,
                        lse, delta, dq, dk, dv, stream);
}

extern "C" int lh_attn_bwd_dkdv(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                                const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                                int split, const int32_t* indices, int B, int H, int n, int D, float scale,
                                const void* dout, const float* lse, const float* delta, void* dk, void* dv,
                                void* stream) {
  return attn_bwd_parts(1, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale, dout,
                        lse, delta, nullptr, dk, dv, stream);
}

extern "C" int lh_attn_bwd_dq(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                              const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                              int split, const int32_t* indices, int B, int H, int n, int D, float scale,
                              const void* dout, const float* lse, const float* delta, void* dq, void* stream) {
  return attn_bwd_parts(2, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale, dout,
                        lse, delta, dq, nullptr, nullptr, stream);
}

extern "C" int lh_dilated_scores(const void* xq, const void* xk, const void* xv, float* scores_qk, float* scores_kq,
                                 int B, int S, int H, int D, int dilation, int S_tot, void* stream) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!xq || !xk || !xv || !scores_qk || !scores_kq || dilation <= 0 || S <= 0 || S % dilation || S_tot < S)
    return LH_ERR_INVALID_ARG;
  const int n = S / dilation;
  const int VH = dilation * H;
  const int64_t sb = (int64_t)S * H * D, ss = (int64_t)VH * D, sh = D;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  for (int pass = 0; pass < 2; ++pass) {
    const void* qq = pass == 0 ? xq : xk;
    const void* kk = pass == 0 ? xk : xq;
    AttnArgs a{};
    int rc = fill_rows(a, qq, kk, xv, sb, ss, sh, nullptr, nullptr, nullptr, 0, 0, 0, 0, nullptr, B, VH, n, D,
                       (float)(1.0 / 11.313708498984761));
    if (rc) return rc;
    a.scores = pass == 0 ? scores_qk : scores_kq;
    a.Ho = H; a.dil = dilation; a.S_tot = S_tot;
    hipLaunchKernelGGL(attn_fwd_kernel<1>, dim3(a.nq * a.BH), dim3(64 * QW), 0, st, a);
    LH_CHECK_LAUNCH();
  }
  return LH_OK;
}

// Causal attention over gathered rows on gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Replaces the three torch.gather calls and the inner causal SDPA of
// LighthouseLocal.forward (src/lighthouse_selection.py:800-815) and, with an
// identity row map and a norm epilogue, the two SDPA calls of
// DilatedLighthouseScorer.forward (:642-653).
//
// Layout choices (one 64-lane wave computes 32 queries x 64 keys per step):
//   * Scores are formed transposed, S^T = K Q^T, so an MFMA output column is a
//     query: lane l holds query l%32 and 16 keys per 32x32 block.  Row max and
//     row sum of the online softmax are in-lane plus one exchange with lane
//     l^32, and the per-query rescale of O is a per-lane scalar.
//   * The exp'd scores feed P V directly from registers: the C-layout of S^T
//     (key = 8*(v/4) + 4*(l/32) + v%4) is used as the k-order of the next MFMA,
//     and V is staged transposed in LDS so the A operand reads the same key
//     order (two 8-byte LDS reads per operand).
//   * Rows are gathered on the fly: row s of (b, h) is read through
//     indices[b, h, s] from the base [B, S, H, D] tensor or the pooled
//     [B, Sp, H, D] tensor; nothing is materialised.
//   * K/V tiles are double-buffered in LDS; the next tile's global loads are
//     issued before the current tile's MFMAs.
//   * Backward is deterministic: dK/dV in a key-stationary kernel, dQ in a
//     query-stationary kernel, no atomics.
// Softmax runs in the exp2 domain with scale*log2(e); the stored LSE is
// m + log2(l) in that domain.
#include "lh_common.h"

namespace {

constexpr int BM = 128;  // queries (or keys) per workgroup: 4 waves x 32
constexpr int BN = 64;   // rows per LDS tile
constexpr int RS = 136;  // row-major tile stride in bf16 (128 + 8 pad)
constexpr int TS = 68;   // transposed tile stride in bf16 (64 + 4 pad)

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

__device__ __forceinline__ floatx16 mfma(const u32x4 a, const u32x4 b, const floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

__device__ __forceinline__ uint32_t cvt2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// element offset of row s of (b, h); `pooled` tells which tensor holds it
__device__ __forceinline__ int64_t row_off(const Rows& R, int b, int h, int bh, int n, int s, bool& pooled) {
  const int r = R.idx ? R.idx[(int64_t)bh * n + s] : s;
  pooled = r >= R.split;
  return pooled ? (int64_t)b * R.pb + (int64_t)(r - R.split) * R.ps + (int64_t)h * R.ph
                : (int64_t)b * R.sb + (int64_t)r * R.ss + (int64_t)h * R.sh;
}

// Blocks are dispatched round-robin over the 8 XCDs; give each XCD a
// contiguous run of (b, h) so K/V rows stay in that XCD's L2, and run the
// heaviest (latest) query blocks first.
__device__ __forceinline__ void schedule(int w, int nblk, int BH, int& bh, int& blk, bool heavy_last) {
  const int total = nblk * BH;
  int t = w;
  if ((total & 7) == 0) t = (w & 7) * (total >> 3) + (w >> 3);
  bh = t / nblk;
  const int r = t % nblk;
  blk = heavy_last ? (nblk - 1 - r) : r;
}

// Tile loader: thread owns rows 4*rq .. 4*rq+3 of the tile and 8 columns at 8*dc.
struct Tile4 {
  u32x4 r[4];
};

__device__ __forceinline__ void load_gathered(Tile4& t, const bf16_t* base, const bf16_t* pool, const Rows& R, int b,
                                              int h, int bh, int n, int row0, int dc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = row0 + i;
    if (s < n) {
      bool pooled;
      const int64_t o = row_off(R, b, h, bh, n, s, pooled);
      t.r[i] = *reinterpret_cast<const u32x4*>((pooled ? pool : base) + o + 8 * dc);
    } else {
      t.r[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

__device__ __forceinline__ void load_dense(Tile4& t, const bf16_t* base, int n, int row0, int dc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = row0 + i;
    t.r[i] = (s < n) ? *reinterpret_cast<const u32x4*>(base + (int64_t)s * LH_D + 8 * dc) : u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void store_rowmajor(const Tile4& t, bf16_t* lds, int rq, int dc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(lds + (4 * rq + i) * RS + 8 * dc) = t.r[i];
}

// lds is [D][TS]: column block of 4 consecutive rows per 8-byte store
__device__ __forceinline__ void store_transposed(const Tile4& t, bf16_t* lds, int rq, int dc) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int w = e >> 1;
    uint32_t a0 = t.r[0][w], a1 = t.r[1][w], a2 = t.r[2][w], a3 = t.r[3][w];
    u32x2 v;
    if (e & 1) {
      v.x = (a0 >> 16) | (a1 & 0xffff0000u);
      v.y = (a2 >> 16) | (a3 & 0xffff0000u);
    } else {
      v.x = (a0 & 0xffffu) | (a1 << 16);
      v.y = (a2 & 0xffffu) | (a3 << 16);
    }
    *reinterpret_cast<u32x2*>(lds + (8 * dc + e) * TS + 4 * rq) = v;
  }
}

// A operand from a transposed tile: row `d`, 16-column chunk starting at col0,
// key order 4*hh + {0..3} then 8 + 4*hh + {0..3}
__device__ __forceinline__ u32x4 ld_tr(const bf16_t* lds, int d, int col0, int hh) {
  const bf16_t* p = lds + d * TS + col0 + 4 * hh;
  const u32x2 lo = *reinterpret_cast<const u32x2*>(p);
  const u32x2 hi = *reinterpret_cast<const u32x2*>(p + 8);
  return u32x4{lo.x, lo.y, hi.x, hi.y};
}

__device__ __forceinline__ u32x4 ld_row(const bf16_t* lds, int row, int col) {
  return *reinterpret_cast<const u32x4*>(lds + row * RS + col);
}

// 8 fp32 accumulator values v = 8*c2 .. 8*c2+7 -> bf16 B operand
__device__ __forceinline__ u32x4 pack_frag(const floatx16& s, int c2) {
  const int v = 8 * c2;
  return u32x4{cvt2(s[v + 0], s[v + 1]), cvt2(s[v + 2], s[v + 3]), cvt2(s[v + 4], s[v + 5]), cvt2(s[v + 6], s[v + 7])};
}

// ===========================================================================
// forward (query-stationary)
// ===========================================================================
template <int EPI>  // 0: O + LSE;  1: bf16-rounded row norms of O into `scores`
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][BN * RS];
  __shared__ __attribute__((aligned(16))) bf16_t Vt[2][LH_D * TS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  int bh, qb;
  schedule(blockIdx.x, a.nq, a.BH, bh, qb, true);
  const int b = bh / a.H, h = bh % a.H, n = a.n;
  const Rows& R = a.R;
  const int q0 = qb * BM, qw = q0 + wave * 32, my_q = qw + l32;

  u32x4 qf[8];
  if (my_q < n) {
    bool pooled;
    const int64_t o = row_off(R, b, h, bh, n, my_q, pooled);
    const bf16_t* p = (pooled ? R.qp : R.q) + o + 8 * hh;
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = *reinterpret_cast<const u32x4*>(p + 16 * c);
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) qf[c] = u32x4{0u, 0u, 0u, 0u};
  }

  const int kend = min(q0 + BM, n);
  const int nt = (kend + BN - 1) / BN;
  const int rq = tid & 15, dc = tid >> 4;
  Tile4 kr, vr;
  load_gathered(kr, R.k, R.kp, R, b, h, bh, n, 4 * rq, dc);
  load_gathered(vr, R.v, R.vp, R, b, h, bh, n, 4 * rq, dc);
  store_rowmajor(kr, Ks[0], rq, dc);
  store_transposed(vr, Vt[0], rq, dc);
  __syncthreads();

  floatx16 o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = floatx16{};
  float m_i = -INFINITY, l_i = 0.f;

  for (int j = 0; j < nt; ++j) {
    const int cur = j & 1;
    const int k0 = j * BN;
    if (j + 1 < nt) {
      load_gathered(kr, R.k, R.kp, R, b, h, bh, n, k0 + BN + 4 * rq, dc);
      load_gathered(vr, R.v, R.vp, R, b, h, bh, n, k0 + BN + 4 * rq, dc);
    }
    if (k0 <= qw + 31) {
      floatx16 s[2] = {floatx16{}, floatx16{}};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) s[kb] = mfma(ld_row(Ks[cur], kb * 32 + l32, 16 * c + 8 * hh), qf[c], s[kb]);
      }
      const bool diag = (k0 + BN - 1 > qw) || (k0 + BN > n);
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float x = s[kb][v] * a.sl2;
          if (diag) {
            const int key = k0 + kb * 32 + 8 * (v >> 2) + 4 * hh + (v & 3);
            if (key > my_q || key >= n) x = -INFINITY;
          }
          s[kb][v] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_i, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = ex2(m_i - m_use);
      float ls = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float pv = ex2(s[kb][v] - m_use);
          s[kb][v] = pv;
          ls += pv;
        }
      }
      ls += __shfl_xor(ls, 32);
      l_i = l_i * alpha + ls;
      m_i = m_new;
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] *= alpha;
      u32x4 pf[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        pf[kb][0] = pack_frag(s[kb], 0);
        pf[kb][1] = pack_frag(s[kb], 1);
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2) o[d] = mfma(ld_tr(Vt[cur], d * 32 + l32, kb * 32 + 16 * c2, hh), pf[kb][c2], o[d]);
        }
      }
    }
    if (j + 1 < nt) {
      store_rowmajor(kr, Ks[cur ^ 1], rq, dc);
      store_transposed(vr, Vt[cur ^ 1], rq, dc);
    }
    __syncthreads();
  }

  if (my_q >= n) return;
  const float inv_l = l_i > 0.f ? 1.0f / l_i : 0.f;
  if (EPI == 0) {
    bf16_t* orow = a.out + ((int64_t)bh * n + my_q) * LH_D;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w.x = cvt2(o[d][4 * g + 0] * inv_l, o[d][4 * g + 1] * inv_l);
        w.y = cvt2(o[d][4 * g + 2] * inv_l, o[d][4 * g + 3] * inv_l);
        *reinterpret_cast<u32x2*>(orow + d * 32 + 8 * g + 4 * hh) = w;
      }
    }
    if (hh == 0) a.lse[(int64_t)bh * n + my_q] = l_i > 0.f ? m_i + __log2f(l_i) : -INFINITY;
  } else {
    float ss = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const uint32_t w = cvt2(o[d][v] * inv_l, o[d][v + 1] * inv_l);
        const float x0 = __uint_as_float(w << 16), x1 = __uint_as_float(w & 0xffff0000u);
        ss = fmaf(x0, x0, ss);
        ss = fmaf(x1, x1, ss);
      }
    }
    ss += __shfl_xor(ss, 32);
    if (hh == 0) {
      const int vh = h;  // virtual head
      const int t = my_q * a.dil + vh / a.Ho;
      const int ho = vh % a.Ho;
      a.scores[((int64_t)b * a.Ho + ho) * a.S_tot + t] = __uint_as_float(cvt2(sqrtf(ss), 0.f) << 16);
    }
  }
}

// ===========================================================================
// backward dQ (query-stationary)
// ===========================================================================
__global__ __launch_bounds__(256, 1) void attn_bwd_dq_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][BN * RS];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[2][BN * RS];
  __shared__ __attribute__((aligned(16))) bf16_t Kt[2][LH_D * TS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  int bh, qb;
  schedule(blockIdx.x, a.nq, a.BH, bh, qb, true);
  const int b = bh / a.H, h = bh % a.H, n = a.n;
  const Rows& R = a.R;
  const int q0 = qb * BM, qw = q0 + wave * 32, my_q = qw + l32;

  u32x4 qf[8], df[8];
  float lse2 = 0.f, dlt = 0.f;
  if (my_q < n) {
    bool pooled;
    const int64_t o = row_off(R, b, h, bh, n, my_q, pooled);
    const bf16_t* p = (pooled ? R.qp : R.q) + o + 8 * hh;
    const bf16_t* pd = a.dout + ((int64_t)bh * n + my_q) * LH_D + 8 * hh;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      qf[c] = *reinterpret_cast<const u32x4*>(p + 16 * c);
      df[c] = *reinterpret_cast<const u32x4*>(pd + 16 * c);
    }
    lse2 = a.lse_in[(int64_t)bh * n + my_q];
    dlt = a.delta[(int64_t)bh * n + my_q];
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) { qf[c] = u32x4{0u, 0u, 0u, 0u}; df[c] = u32x4{0u, 0u, 0u, 0u}; }
  }

  const int kend = min(q0 + BM, n);
  const int nt = (kend + BN - 1) / BN;
  const int rq = tid & 15, dc = tid >> 4;
  Tile4 kr, vr;
  load_gathered(kr, R.k, R.kp, R, b, h, bh, n, 4 * rq, dc);
  load_gathered(vr, R.v, R.vp, R, b, h, bh, n, 4 * rq, dc);
  store_rowmajor(kr, Ks[0], rq, dc);
  store_transposed(kr, Kt[0], rq, dc);
  store_rowmajor(vr, Vs[0], rq, dc);
  __syncthreads();

  floatx16 acc[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) acc[d] = floatx16{};

  for (int j = 0; j < nt; ++j) {
    const int cur = j & 1;
    const int k0 = j * BN;
    if (j + 1 < nt) {
      load_gathered(kr, R.k, R.kp, R, b, h, bh, n, k0 + BN + 4 * rq, dc);
      load_gathered(vr, R.v, R.vp, R, b, h, bh, n, k0 + BN + 4 * rq, dc);
    }
    if (k0 <= qw + 31) {
      floatx16 s[2] = {floatx16{}, floatx16{}}, dp[2] = {floatx16{}, floatx16{}};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          s[kb] = mfma(ld_row(Ks[cur], kb * 32 + l32, 16 * c + 8 * hh), qf[c], s[kb]);
          dp[kb] = mfma(ld_row(Vs[cur], kb * 32 + l32, 16 * c + 8 * hh), df[c], dp[kb]);
        }
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + kb * 32 + 8 * (v >> 2) + 4 * hh + (v & 3);
          const bool masked = key > my_q || key >= n || my_q >= n;
          const float p = masked ? 0.f : ex2(s[kb][v] * a.sl2 - lse2);
          s[kb][v] = p * (dp[kb][v] - dlt);
        }
      }
      u32x4 sf[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sf[kb][0] = pack_frag(s[kb], 0);
        sf[kb][1] = pack_frag(s[kb], 1);
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2)
            acc[d] = mfma(ld_tr(Kt[cur], d * 32 + l32, kb * 32 + 16 * c2, hh), sf[kb][c2], acc[d]);
        }
      }
    }
    if (j + 1 < nt) {
      store_rowmajor(kr, Ks[cur ^ 1], rq, dc);
      store_transposed(kr, Kt[cur ^ 1], rq, dc);
      store_rowmajor(vr, Vs[cur ^ 1], rq, dc);
    }
    __syncthreads();
  }

  if (my_q >= n) return;
  bf16_t* orow = a.dq + ((int64_t)bh * n + my_q) * LH_D;
  const float sc = a.scale;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w.x = cvt2(acc[d][4 * g + 0] * sc, acc[d][4 * g + 1] * sc);
      w.y = cvt2(acc[d][4 * g + 2] * sc, acc[d][4 * g + 3] * sc);
      *reinterpret_cast<u32x2*>(orow + d * 32 + 8 * g + 4 * hh) = w;
    }
  }
}

// ===========================================================================
// backward dK, dV (key-stationary)
// ===========================================================================
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t Qs[2][BN * RS];
  __shared__ __attribute__((aligned(16))) bf16_t Ds[2][BN * RS];
  __shared__ __attribute__((aligned(16))) bf16_t Qt[2][LH_D * TS];
  __shared__ __attribute__((aligned(16))) bf16_t Dt[2][LH_D * TS];
  __shared__ __attribute__((aligned(16))) float Ls[2][BN];
  __shared__ __attribute__((aligned(16))) float Dl[2][BN];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  int bh, kblk;
  schedule(blockIdx.x, a.nq, a.BH, bh, kblk, false);  // early key blocks see the most queries
  const int b = bh / a.H, h = bh % a.H, n = a.n;
  const Rows& R = a.R;
  const int k0 = kblk * BM, kw = k0 + wave * 32, my_k = kw + l32;

  u32x4 kf[8], vf[8];
  if (my_k < n) {
    bool pooled;
    const int64_t o = row_off(R, b, h, bh, n, my_k, pooled);
    const bf16_t* pk = (pooled ? R.kp : R.k) + o + 8 * hh;
    const bf16_t* pv = (pooled ? R.vp : R.v) + o + 8 * hh;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      kf[c] = *reinterpret_cast<const u32x4*>(pk + 16 * c);
      vf[c] = *reinterpret_cast<const u32x4*>(pv + 16 * c);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) { kf[c] = u32x4{0u, 0u, 0u, 0u}; vf[c] = u32x4{0u, 0u, 0u, 0u}; }
  }

  const int jt0 = k0 / BN;
  const int nt = (n + BN - 1) / BN;
  const int rq = tid & 15, dc = tid >> 4;
  const bf16_t* dbase = a.dout + (int64_t)bh * n * LH_D;
  const float* lrow = a.lse_in + (int64_t)bh * n;
  const float* drow = a.delta + (int64_t)bh * n;
  Tile4 qr, dr;
  float lv = 0.f;
  {
    const int q0t = jt0 * BN;
    load_gathered(qr, R.q, R.qp, R, b, h, bh, n, q0t + 4 * rq, dc);
    load_dense(dr, dbase, n, q0t + 4 * rq, dc);
    if (tid < 2 * BN) {
      const int qq = q0t + (tid & (BN - 1));
      lv = qq < n ? (tid < BN ? lrow[qq] : drow[qq]) : 0.f;
    }
    store_rowmajor(qr, Qs[0], rq, dc);
    store_transposed(qr, Qt[0], rq, dc);
    store_rowmajor(dr, Ds[0], rq, dc);
    store_transposed(dr, Dt[0], rq, dc);
    if (tid < BN) Ls[0][tid] = lv; else if (tid < 2 * BN) Dl[0][tid - BN] = lv;
  }
  __syncthreads();

  floatx16 dka[4], dva[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) { dka[d] = floatx16{}; dva[d] = floatx16{}; }

  for (int j = jt0; j < nt; ++j) {
    const int cur = (j - jt0) & 1;
    const int q0t = j * BN;
    if (j + 1 < nt) {
      const int qn = q0t + BN;
      load_gathered(qr, R.q, R.qp, R, b, h, bh, n, qn + 4 * rq, dc);
      load_dense(dr, dbase, n, qn + 4 * rq, dc);
      if (tid < 2 * BN) {
        const int qq = qn + (tid & (BN - 1));
        lv = qq < n ? (tid < BN ? lrow[qq] : drow[qq]) : 0.f;
      }
    }
    if (q0t + BN - 1 >= kw) {
      floatx16 s[2] = {floatx16{}, floatx16{}}, dp[2] = {floatx16{}, floatx16{}};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          s[qb] = mfma(ld_row(Qs[cur], qb * 32 + l32, 16 * c + 8 * hh), kf[c], s[qb]);
          dp[qb] = mfma(ld_row(Ds[cur], qb * 32 + l32, 16 * c + 8 * hh), vf[c], dp[qb]);
        }
      }
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int qi = qb * 32 + 8 * g + 4 * hh;
          const float4 l4 = *reinterpret_cast<const float4*>(&Ls[cur][qi]);
          const float4 d4 = *reinterpret_cast<const float4*>(&Dl[cur][qi]);
          const float lq[4] = {l4.x, l4.y, l4.z, l4.w};
          const float dq4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int v = 4 * g + e;
            const int q = q0t + qi + e;
            const bool masked = my_k > q || q >= n || my_k >= n;
            const float p = masked ? 0.f : ex2(s[qb][v] * a.sl2 - lq[e]);
            s[qb][v] = p;
            dp[qb][v] = p * (dp[qb][v] - dq4[e]);
          }
        }
      }
      u32x4 pf[2][2], sf[2][2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        pf[qb][0] = pack_frag(s[qb], 0);
        pf[qb][1] = pack_frag(s[qb], 1);
        sf[qb][0] = pack_frag(dp[qb], 0);
        sf[qb][1] = pack_frag(dp[qb], 1);
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
          for (int c2 = 0; c2 < 2; ++c2) {
            dva[d] = mfma(ld_tr(Dt[cur], d * 32 + l32, qb * 32 + 16 * c2, hh), pf[qb][c2], dva[d]);
            dka[d] = mfma(ld_tr(Qt[cur], d * 32 + l32, qb * 32 + 16 * c2, hh), sf[qb][c2], dka[d]);
          }
        }
      }
    }
    if (j + 1 < nt) {
      store_rowmajor(qr, Qs[cur ^ 1], rq, dc);
      store_transposed(qr, Qt[cur ^ 1], rq, dc);
      store_rowmajor(dr, Ds[cur ^ 1], rq, dc);
      store_transposed(dr, Dt[cur ^ 1], rq, dc);
      if (tid < BN) Ls[cur ^ 1][tid] = lv; else if (tid < 2 * BN) Dl[cur ^ 1][tid - BN] = lv;
    }
    __syncthreads();
  }

  if (my_k >= n) return;
  bf16_t* krow = a.dk + ((int64_t)bh * n + my_k) * LH_D;
  bf16_t* vrow = a.dv + ((int64_t)bh * n + my_k) * LH_D;
  const float sc = a.scale;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w.x = cvt2(dka[d][4 * g + 0] * sc, dka[d][4 * g + 1] * sc);
      w.y = cvt2(dka[d][4 * g + 2] * sc, dka[d][4 * g + 3] * sc);
      *reinterpret_cast<u32x2*>(krow + d * 32 + 8 * g + 4 * hh) = w;
      w.x = cvt2(dva[d][4 * g + 0], dva[d][4 * g + 1]);
      w.y = cvt2(dva[d][4 * g + 2], dva[d][4 * g + 3]);
      *reinterpret_cast<u32x2*>(vrow + d * 32 + 8 * g + 4 * hh) = w;
    }
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int fill_rows(AttnArgs& a, const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
              const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph, int split,
              const int32_t* indices, int B, int H, int n, int D, float scale) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!q || !k || !v || B <= 0 || H <= 0 || n <= 0) return LH_ERR_INVALID_ARG;
  if (!al16(q) || !al16(k) || !al16(v) || (sb | ss | sh) % 8) return LH_ERR_INVALID_ARG;
  const bool need_pool = indices != nullptr;  // pooled rows only reachable through an index map
  if (need_pool && (!qp || !kp || !vp || !al16(qp) || !al16(kp) || !al16(vp) || (pb | ps | ph) % 8))
    return LH_ERR_INVALID_ARG;
  if (!(scale > 0.f)) return LH_ERR_INVALID_ARG;
  a.R.q = (const bf16_t*)q; a.R.k = (const bf16_t*)k; a.R.v = (const bf16_t*)v;
  a.R.qp = (const bf16_t*)(qp ? qp : q); a.R.kp = (const bf16_t*)(kp ? kp : k); a.R.vp = (const bf16_t*)(vp ? vp : v);
  a.R.sb = sb; a.R.ss = ss; a.R.sh = sh; a.R.pb = pb; a.R.ps = ps; a.R.ph = ph;
  a.R.split = indices ? split : 0x7fffffff;
  a.R.idx = indices;
  a.B = B; a.H = H; a.n = n; a.BH = B * H;
  a.nq = (n + BM - 1) / BM;
  a.scale = scale;
  a.sl2 = (float)((double)scale * 1.4426950408889634);
  if ((long long)a.nq * a.BH > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
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
  hipLaunchKernelGGL(attn_fwd_kernel<0>, dim3(a.nq * a.BH), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
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
    hipLaunchKernelGGL(attn_bwd_dkdv_kernel, dim3(a.nq * a.BH), dim3(256), 0, st, a);
    LH_CHECK_LAUNCH();
  }
  if (parts & 2) {
    hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3(a.nq * a.BH), dim3(256), 0, st, a);
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
    hipLaunchKernelGGL(attn_fwd_kernel<1>, dim3(a.nq * a.BH), dim3(256), 0, st, a);
    LH_CHECK_LAUNCH();
  }
  return LH_OK;
}

// Hierarchical per-tile top-k selection for gfx950.
//
// One 4-wave workgroup per (b, h, tile).  The 128-element working set of the
// reference block (src/lighthouse_selection_cuda.py:150-157) lives in the
// registers of one wave: element e = 64*slot + lane.  Compare-exchanges at
// distance 64 are in-lane; distances 1..32 are cross-lane shuffles.  Wave 0
// runs the qk sorts and wave 1 the kq sorts, one batch behind, the qk rejects
// handed over in LDS; all four waves load candidates, rank and emit.  The network, the batch
// structure and the candidate order follow src/lighthouse_selection_cuda.py:
//   - sort network:                 :41-110 (strict compare-exchange)
//   - candidates (coarsest/children): :177-229
//   - qk then kq streaming sorts:     :232-258
//   - selected = [TQ | TK], parents:  :274-289, :324-327
//
// Output order.  The reference emits every valid candidate once (as a kq
// reject, as one of the final [TQ | TK], or as a level-1 leaf) with an
// order key, then sorts the keys (:11-25, :425-427).  Here the emitted set is
// taken structurally (every candidate of every level, flagged selected or
// not), each entry's integer key (key * 2^(L-1)) is set in an LDS bitmap over
// the tile's key span, and an entry's output position is its rank among the
// set bits.  Tiles own disjoint key ranges, so the result is tile-major and no
// global sort is needed.  The same pass writes the inverse map
// (pyramid index -> selected position, -1 elsewhere) for the tile's pyramid
// ranges; the last tile also clears the trailing nodes no tile visits.
#include "lh_common.h"

namespace {

constexpr int TOPK = 128;
constexpr int HALF = 64;
constexpr float SENT = -1e6f;

struct SelParams {
  int S, L, p, shift, T, NCC, per_tile, S_sel, S_tot;
  int nc_pad;             // candidate slots per level, padded to 64
  int off[9], len[9];     // pyramid level offsets and lengths
  int R[9];               // nodes of level l inside one tile
  int selw_off[9];        // word offset of level l's selected bitmask (l >= 2)
  int sel_words;          // total selected-bitmask words
  int key_words;          // words of the key bitmap
  int lds_bytes;
};

// ---------------------------------------------------------------------------
// Value of lane ^ J without a round trip through LDS: DPP quad permutes for 1
// and 2, a half-row mirror followed by a quad reversal for 4, a 16-lane row
// rotation by 8 for 8, the gfx950 row/half swaps for 16 and 32.
// ---------------------------------------------------------------------------
template <int J>
__device__ __forceinline__ int lane_xor(int v, int lane) {
  if constexpr (J == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
  else if constexpr (J == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);  // quad_perm [2,3,0,1]
  else if constexpr (J == 4)  // row_half_mirror (i -> 7 - i in each 8 lanes), then quad_perm [3,2,1,0]
    return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF, true);
  else if constexpr (J == 8) return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, true);  // row_ror:8
  else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? (int)r[0] : (int)r[1];
  } else {
    static_assert(J == 32, "lane distance");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? (int)r[0] : (int)r[1];
  }
}

// ---------------------------------------------------------------------------
// compare-exchange at lane distance J (1..32) for one slot
// ---------------------------------------------------------------------------
template <int TIE, int J>
__device__ __forceinline__ void cx_lane(float& s, int& x, int& id, bool desc, int lane) {
  const float os = __int_as_float(lane_xor<J>(__float_as_int(s), lane));
  const int ox = lane_xor<J>(x, lane);
  const int oid = TIE ? lane_xor<J>(id, lane) : 0;
  const int j = J;
  const bool keep_max = (((lane & j) == 0) == desc);
  // take = keep_max ? (s < os) : (s > os), as one compare of a lane-ordered
  // pair (a, b) = keep_max ? (s, os) : (os, s): take = a < b
  const float a = keep_max ? s : os, b = keep_max ? os : s;
  bool take;
  if (TIE == LH_TIE_REFERENCE) {
    take = a < b;
  } else {
    // other_better on keep_max lanes, mine_better elsewhere: b beats a on the
    // score, or ties with a smaller id (-1 -> largest: invalid ids lose ties)
    const unsigned mk = (unsigned)id, ok = (unsigned)oid;
    const unsigned ai = keep_max ? mk : ok, bi = keep_max ? ok : mk;
    take = (b > a) || (b == a && bi < ai);
  }
  if (take) { s = os; x = ox; id = oid; }
}

// One stage (k, j) of the descending 128-wide bitonic sort; element e = 64*slot + lane.
template <int TIE, int K, int J>
__device__ __forceinline__ void sort_stage(float& s0, int& x0, int& i0, float& s1, int& x1, int& i1, int lane) {
  if constexpr (J == 64) {  // k == 128: pair (lane, 64 + lane), descending
    bool take;
    if (TIE == LH_TIE_REFERENCE) {
      take = s0 < s1;
    } else {
      take = (s1 > s0) || (s1 == s0 && (unsigned)i1 < (unsigned)i0);
    }
    if (take) {
      float ts = s0; s0 = s1; s1 = ts;
      int tx = x0; x0 = x1; x1 = tx;
      int ti = i0; i0 = i1; i1 = ti;
    }
  } else {
    const bool desc0 = (K >= 64) ? true : ((lane & K) == 0);
    const bool desc1 = (K == 128) ? true : (K == 64 ? false : ((lane & K) == 0));
    cx_lane<TIE, J>(s0, x0, i0, desc0, lane);
    cx_lane<TIE, J>(s1, x1, i1, desc1, lane);
  }
  if constexpr (J > 1) sort_stage<TIE, K, J / 2>(s0, x0, i0, s1, x1, i1, lane);
}

template <int TIE, int K>
__device__ __forceinline__ void sort_from(float& s0, int& x0, int& i0, float& s1, int& x1, int& i1, int lane) {
  sort_stage<TIE, K, K / 2>(s0, x0, i0, s1, x1, i1, lane);
  if constexpr (K < TOPK) sort_from<TIE, 2 * K>(s0, x0, i0, s1, x1, i1, lane);
}

// Descending 128-wide bitonic sort; element e = 64*slot + lane.
template <int TIE>
__device__ __forceinline__ void sort128(float& s0, int& x0, int& i0, float& s1, int& x1, int& i1, int lane) {
  sort_from<TIE, 2>(s0, x0, i0, s1, x1, i1, lane);
}

__device__ __forceinline__ bool get_bit(const uint32_t* bits, int i) {
  return (bits[i >> 5] >> (i & 31)) & 1u;
}

template <int TIE>
__global__ __launch_bounds__(256) void select_kernel(const float* __restrict__ sqk,
                                                     const float* __restrict__ skq,
                                                     int32_t* __restrict__ indices,
                                                     int32_t* __restrict__ inverse,
                                                     const SelParams P) {
  const int tile = blockIdx.x;
  const int bh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  extern __shared__ uint32_t smem[];
  float* sc_qk = reinterpret_cast<float*>(smem);
  float* sc_kq = sc_qk + P.nc_pad;
  int* cand = reinterpret_cast<int*>(sc_kq + P.nc_pad);
  int* parent = cand + P.nc_pad;
  int* rej = parent + TOPK;  // [2][64]: qk rejects of a batch, handed from wave 0 to wave 1
  uint32_t* selbits = reinterpret_cast<uint32_t*>(rej + 2 * HALF);
  uint32_t* kbits = selbits + P.sel_words;
  uint32_t* kpre = kbits + P.key_words;

  const float* q = sqk + (size_t)bh * P.S_tot;
  const float* k = skq + (size_t)bh * P.S_tot;
  const int L = P.L, p = P.p, shift = P.shift;

  for (int w = tid; w < P.sel_words; w += 256) selbits[w] = 0u;
  for (int w = tid; w < P.key_words; w += 256) kbits[w] = 0u;
  if (tid < TOPK) parent[tid] = -1;
  __syncthreads();

  // ------------------------------------------------------------------ select
  // Per level, batch b's qk sort (wave 0) and batch b-1's kq sort (wave 1)
  // run side by side: the kq sort of a batch depends on its qk rejects and on
  // the previous kq sort only, so the two streams are the reference's order.
  for (int level = L; level >= 2; --level) {
    const int off = P.off[level];
    const int nc = (level == L) ? P.NCC : p * TOPK;
    const int nb = (nc + HALF - 1) / HALF;
    for (int a = tid; a < nb * HALF; a += 256) {
      int id = -1;
      if (a < nc) {
        if (level == L) {
          id = tile * P.NCC + a;
        } else {
          const int par = parent[a >> shift];
          if (par >= 0) id = par * p + (a & (p - 1));
        }
        if (id >= P.len[level]) id = -1;
      }
      cand[a] = id;
      sc_qk[a] = id >= 0 ? q[off + id] : SENT;
      sc_kq[a] = id >= 0 ? k[off + id] : SENT;
    }
    __syncthreads();

    float t_s = SENT;
    int t_x = -1, t_i = -1;  // TQ (wave 0) or TK (wave 1)
    for (int b = 0; b <= nb; ++b) {
      if (wave == 0 && b < nb) {
        const int a = b * HALF + lane;
        float s0 = t_s, s1 = sc_qk[a];
        int x0 = t_x, x1 = cand[a] >= 0 ? a : -1;
        int i0 = t_i, i1 = TIE ? cand[a] : 0;
        sort128<TIE>(s0, x0, i0, s1, x1, i1, lane);
        t_s = s0; t_x = x0; t_i = i0;
        rej[(b & 1) * HALF + lane] = x1;  // qk rejects (positions 64..127) stream into the kq sort
      } else if (wave == 1 && b >= 1) {
        const int r = rej[((b - 1) & 1) * HALF + lane];
        float u0 = t_s, u1 = r >= 0 ? sc_kq[r] : SENT;
        int y0 = t_x, y1 = r;
        int j0 = t_i, j1 = TIE ? (r >= 0 ? cand[r] : -1) : 0;
        sort128<TIE>(u0, y0, j0, u1, y1, j1, lane);
        t_s = u0; t_x = y0; t_i = j0;
      }
      __syncthreads();
    }
    const int id = (wave < 2 && t_x >= 0) ? cand[t_x] : -1;
    __syncthreads();  // every lane has read parent[] and cand[] for this level
    if (wave < 2) {
      parent[lane + HALF * wave] = id;  // [TQ | TK]
      if (id >= 0) {
        uint32_t* sb = selbits + P.selw_off[level];
        const int t = id - tile * P.R[level];
        atomicOr(&sb[t >> 5], 1u << (t & 31));
      }
    }
    __syncthreads();
  }

  // ------------------------------------------------------------------ rank
  const int kscale_shift = L - 1;
  const long long key_base = (long long)tile * P.NCC * ((long long)1 << ((L - 1) * shift)) << kscale_shift;
  for (int level = L; level >= 1; --level) {
    const int Rl = P.R[level];
    const int base = tile * Rl;
    const int c_shift = (level - 1) * shift;  // log2 c_l
    for (int j = tid; j < Rl; j += 256) {
      const bool is_cand = (level == L) || get_bit(selbits + P.selw_off[level + 1], j >> shift);
      if (!is_cand) continue;
      const bool is_sel = (level >= 2) && get_bit(selbits + P.selw_off[level], j);
      const long long i = base + j;
      const long long key = is_sel ? ((((i + 1) << c_shift) << kscale_shift) - (1LL << (L - level)))
                                   : ((i << c_shift) << kscale_shift);
      const int rel = (int)(key - key_base);
      atomicOr(&kbits[rel >> 5], 1u << (rel & 31));
    }
  }
  __syncthreads();
  if (wave == 0) {  // exclusive prefix of popcounts per key word
    const int chunk = (P.key_words + 63) / 64;
    const int w0 = lane * chunk;
    const int w1 = min(w0 + chunk, P.key_words);
    int local = 0;
    for (int w = w0; w < w1; ++w) local += __popc(kbits[w]);
    int incl = local;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    int run = incl - local;
    for (int w = w0; w < w1; ++w) { kpre[w] = (uint32_t)run; run += __popc(kbits[w]); }
  }
  __syncthreads();

  // ------------------------------------------------------------------ emit
  int32_t* out = indices + (size_t)bh * P.S_sel + (size_t)tile * P.per_tile;
  int32_t* inv = inverse ? inverse + (size_t)bh * P.S_tot : nullptr;
  for (int level = L; level >= 1; --level) {
    const int Rl = P.R[level];
    const int base = tile * Rl;
    const int c_shift = (level - 1) * shift;
    // the last tile also owns the trailing nodes that no tile visits
    const int jend = (inv && tile == P.T - 1) ? (P.len[level] - base) : Rl;
    for (int j = tid; j < jend; j += 256) {
      int pos = -1;
      if (j < Rl) {
        const bool is_cand = (level == L) || get_bit(selbits + P.selw_off[level + 1], j >> shift);
        if (is_cand) {
          const bool is_sel = (level >= 2) && get_bit(selbits + P.selw_off[level], j);
          const long long i = base + j;
          const long long key = is_sel ? ((((i + 1) << c_shift) << kscale_shift) - (1LL << (L - level)))
                                       : ((i << c_shift) << kscale_shift);
          const int rel = (int)(key - key_base);
          const int rank = (int)kpre[rel >> 5] + __popc(kbits[rel >> 5] & ((1u << (rel & 31)) - 1u));
          if (rank < P.per_tile) {
            out[rank] = P.off[level] + base + j;
            pos = tile * P.per_tile + rank;
          }
        }
      }
      if (inv) inv[P.off[level] + base + j] = pos;
    }
  }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, size_t n, int32_t v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

__global__ void inverse_scatter_kernel(const int32_t* __restrict__ idx, int n, int32_t* __restrict__ inv,
                                       int S_tot, int BH) {
  const size_t total = (size_t)BH * n;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int bh = (int)(i / n), s = (int)(i % n);
    const int r = idx[i];
    if (r >= 0 && r < S_tot) inv[(size_t)bh * S_tot + r] = s;
  }
}

// Geometry shared by the host entry points.
int geometry(int S, int L, int p, int topk, int strict, int* T, int* NCC, int* per_tile, int* S_sel,
             Pyramid* pyr) {
  if (L < 2 || L > 8 || p < 2 || (p & (p - 1)) || topk < TOPK || topk % TOPK || topk / 2 < p || S <= 0)
    return LH_ERR_INVALID_ARG;
  if (!make_pyramid(S, L, p, pyr)) return LH_ERR_INVALID_ARG;
  const int t = topk / TOPK;
  const int coarsest = pyr->len[L];
  const int ncc = coarsest / t;
  if (ncc < 1) return strict ? LH_ERR_DOMAIN : LH_ERR_INVALID_ARG;
  if (strict) {
    const int cL = ipow(p, L - 1);
    if (ncc < TOPK || ncc % HALF || coarsest % t || S % cL) return LH_ERR_DOMAIN;
  }
  int n = ncc, total = ncc;
  for (int l = L - 1; l >= 1; --l) {
    n = p * (n < TOPK ? n : TOPK);
    total += n;
  }
  *T = t; *NCC = ncc; *per_tile = total;
  *S_sel = t * total;
  return LH_OK;
}

}  // namespace

extern "C" int lh_select_geometry(int S, int L, int p, int topk, int strict,
                                  int* num_tiles, int* nodes_per_tile, int* per_tile, int* S_sel) {
  int T, NCC, pt, ss;
  Pyramid g;
  const int rc = geometry(S, L, p, topk, strict, &T, &NCC, &pt, &ss, &g);
  if (rc) return rc;
  if (num_tiles) *num_tiles = T;
  if (nodes_per_tile) *nodes_per_tile = NCC;
  if (per_tile) *per_tile = pt;
  if (S_sel) *S_sel = ss;
  return LH_OK;
}

extern "C" int lh_select_topk(const float* scores_qk, const float* scores_kq, int32_t* indices,
                              int32_t* inverse, int B, int H, int S, int L, int p, int topk,
                              int tie_mode, int strict, void* stream) {
  if (!scores_qk || !scores_kq || !indices || B <= 0 || H <= 0) return LH_ERR_INVALID_ARG;
  if (tie_mode != LH_TIE_REFERENCE && tie_mode != LH_TIE_LOWER_INDEX) return LH_ERR_INVALID_ARG;
  SelParams P{};
  Pyramid g;
  int rc = geometry(S, L, p, topk, strict, &P.T, &P.NCC, &P.per_tile, &P.S_sel, &g);
  if (rc) return rc;
  if ((long long)B * H > 65535 || P.T > 2147483647) return LH_ERR_UNSUPPORTED;
  P.S = S; P.L = L; P.p = p; P.shift = ilog2_exact(p); P.S_tot = g.total;
  for (int l = 1; l <= L; ++l) { P.off[l] = g.off[l]; P.len[l] = g.len[l]; }
  const int ncmax = P.NCC > p * TOPK ? P.NCC : p * TOPK;
  P.nc_pad = (ncmax + HALF - 1) / HALF * HALF;
  int words = 0;
  for (int l = L; l >= 1; --l) {
    P.R[l] = P.NCC * ipow(p, L - l);
    P.selw_off[l] = words;
    if (l >= 2) words += (P.R[l] + 31) / 32;
  }
  P.sel_words = words;
  // key span of one tile: NCC * c_L * 2^(L-1) integer keys
  const long long span = (long long)P.NCC * ipow(p, L - 1) * (1LL << (L - 1));
  if ((long long)S * ipow(p, 0) * (1LL << (L - 1)) >= (1LL << 31)) return LH_ERR_UNSUPPORTED;
  P.key_words = (int)((span + 31) / 32);
  const long long lds = 4LL * (3LL * P.nc_pad + TOPK + 2 * HALF + P.sel_words + 2LL * P.key_words);
  if (lds > 65536) return LH_ERR_UNSUPPORTED;
  P.lds_bytes = (int)lds;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid(P.T, B * H);
  if (tie_mode == LH_TIE_REFERENCE)
    hipLaunchKernelGGL(select_kernel<LH_TIE_REFERENCE>, grid, dim3(256), P.lds_bytes, st, scores_qk, scores_kq,
                       indices, inverse, P);
  else
    hipLaunchKernelGGL(select_kernel<LH_TIE_LOWER_INDEX>, grid, dim3(256), P.lds_bytes, st, scores_qk, scores_kq,
                       indices, inverse, P);
  LH_CHECK_LAUNCH();
  return LH_OK;
}

extern "C" int lh_build_inverse(const int32_t* indices, int n, int32_t* inverse, int S_tot, int B, int H,
                                void* stream) {
  if (!indices || !inverse || n < 0 || S_tot <= 0 || B <= 0 || H <= 0) return LH_ERR_INVALID_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const size_t tot = (size_t)B * H * S_tot;
  const int blocks = (int)((tot + 255) / 256 < 65536 ? (tot + 255) / 256 : 65536);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks), dim3(256), 0, st, inverse, tot, -1);
  LH_CHECK_LAUNCH();
  if (n > 0) {
    const size_t tn = (size_t)B * H * n;
    const int b2 = (int)((tn + 255) / 256 < 65536 ? (tn + 255) / 256 : 65536);
    hipLaunchKernelGGL(inverse_scatter_kernel, dim3(b2), dim3(256), 0, st, indices, n, inverse, S_tot, B * H);
    LH_CHECK_LAUNCH();
  }
  return LH_OK;
}

// ---------------------------------------------------------------------------
// Index validation (debug aid; the Python layer runs it in its check mode).
// counts[0] += entries outside [lo, hi); with marks, counts[1] += entries whose
// row was already named earlier by the same (b, h) (so counts[1] is the number
// of duplicates: k copies of a row add k - 1).  Negative entries inside the
// range (-1 with lo = -1: an empty slot) are not counted as duplicates.
// ---------------------------------------------------------------------------
__global__ void zero_counts_kernel(int32_t* __restrict__ counts) {
  if (threadIdx.x < 2) counts[threadIdx.x] = 0;
}

__global__ void check_indices_kernel(const int32_t* __restrict__ idx, int n, int BH, int lo, int hi,
                                     int32_t* __restrict__ marks, int32_t* __restrict__ counts) {
  const size_t total = (size_t)BH * n;
  int bad = 0, dup = 0;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int r = idx[i];
    if (r < lo || r >= hi) {
      ++bad;
    } else if (marks && r >= 0) {  // r == -1 (allowed when lo == -1) marks an empty slot
      const size_t bh = i / n;
      if (atomicAdd(&marks[bh * (size_t)(hi - lo) + (r - lo)], 1) != 0) ++dup;
    }
  }
  if (bad) atomicAdd(&counts[0], bad);
  if (dup) atomicAdd(&counts[1], dup);
}

extern "C" int lh_check_indices(const int32_t* indices, int B, int H, int n, int lo, int hi, int32_t* marks,
                                int32_t* counts, void* stream) {
  if (!indices || !counts || B <= 0 || H <= 0 || n < 0 || hi <= lo) return LH_ERR_INVALID_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(zero_counts_kernel, dim3(1), dim3(64), 0, st, counts);
  LH_CHECK_LAUNCH();
  if (marks) {
    const size_t tot = (size_t)B * H * (size_t)(hi - lo);
    const int blocks = (int)((tot + 255) / 256 < 65536 ? (tot + 255) / 256 : 65536);
    hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks), dim3(256), 0, st, marks, tot, 0);
    LH_CHECK_LAUNCH();
  }
  if (n > 0) {
    const size_t tn = (size_t)B * H * n;
    const int b2 = (int)((tn + 255) / 256 < 4096 ? (tn + 255) / 256 : 4096);
    hipLaunchKernelGGL(check_indices_kernel, dim3(b2), dim3(256), 0, st, indices, n, B * H, lo, hi, marks, counts);
    LH_CHECK_LAUNCH();
  }
  return LH_OK;
}

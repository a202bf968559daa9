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

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <thread>
#include <type_traits>
#include <utility>
#include <vector>

namespace {

constexpr int BMK = 128;  // keys per workgroup of the key-stationary kernel: 4 waves x 32
constexpr int QW = 8;     // waves per workgroup of the query-stationary kernels (32 queries each)
constexpr int BN = 64;   // rows per LDS tile
constexpr float RESCALE_LOG2 = 8.0f;
constexpr int FWD_AHEAD = 4;  // forward: LDS operands read this many MFMAs ahead
constexpr int DQ_AHEAD = 4;   // dQ kernel, S and dP products
constexpr int DQ_AHEAD2 = 4;  // dQ kernel, dS K product

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));

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

// The attention kernels run on bf16 or fp16 rows (element type T, BF16 or F16):
// the matrix-core product, the rounding of P / dS / outputs and the row sums of
// the rounded values follow T; everything else is type-free 16-bit data.
template <typename T>
__device__ __forceinline__ floatx16 mfma(const u32x4 a, const u32x4 b, const floatx16 c) {
  if constexpr (std::is_same_v<T, F16>)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

template <typename T>
__device__ __forceinline__ uint32_t cvt2(float lo, float hi) {
  return T::pack2(lo, hi);
}

// two packed 16-bit values as the vector type of the dot builtins (a memcpy:
// this compiler mis-lowers __builtin_bit_cast of a single vector element)
__device__ __forceinline__ bf16x2 as_bf2(uint32_t u) {
  bf16x2 r;
  __builtin_memcpy(&r, &u, 4);
  return r;
}
__device__ __forceinline__ lh_f16x2 as_h2(uint32_t u) {
  lh_f16x2 r;
  __builtin_memcpy(&r, &u, 4);
  return r;
}

// acc + the two values packed in u (exact products with 1, fp32 sum): row sums
// of rounded operands, two terms per v_dot2
template <typename T>
__device__ __forceinline__ float dot2one(uint32_t u, float acc) {
  if constexpr (std::is_same_v<T, F16>)
    return __builtin_amdgcn_fdot2(as_h2(u), as_h2(0x3c003c00u), acc, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(as_bf2(u), as_bf2(0x3f803f80u), acc, false);
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

// Query-block plan of the query-stationary kernels.  Causal query blocks of one
// (b, h) cost 1, 2, .. nq key tiles, and with one (b, h) per XCD the hardware's
// heaviest-first list scheduling leaves about 8% of the XCD's CUs idle at the
// end (72 blocks on 32 CUs at cfg2).  With a plan the grid is one workgroup
// per CU: workgroup w (XCD w % 8) is bin (w / 8) % bph of (b, h)
// 8 ((w / 8) / bph) + w % 8 and runs, one after the other, the query blocks
// blk[bin * ipb + k] (k < ipb, PLAN_NONE = none), packed on the host so that
// every bin carries nearly the same number of key tiles.  bph = 0: no plan
// (work queues or one block per workgroup).  The plan travels in the kernel
// arguments: no device state, so concurrent launches cannot interfere.  Plans
// are used only up to 3.5 blocks per bin: with more blocks per CU the list
// schedule is already balanced, and the packed bins measured slower (dense
// n = 32768: 4 per bin, +0.8%; 5.5 per bin, +5.8%; 16 per bin, +11.5%).
constexpr int QPLAN_MAX = 1024;
constexpr uint16_t PLAN_NONE = 0xffff;
struct QPlan {
  int bph;  // bins (workgroups) per (b, h); 0 = no plan
  int ipb;  // slots per bin
  uint16_t blk[QPLAN_MAX];
};

// (b, h), bin and first query block of this workgroup under a plan
__device__ __forceinline__ void plan_first(const QPlan& p, int& bh, int& bin, int& qb) {
  const int i = blockIdx.x >> 3;
  bh = (i / p.bph) * 8 + (blockIdx.x & 7);
  bin = i % p.bph;
  qb = p.blk[bin * p.ipb];
}

// Query block k of this workgroup's bin (false: none); waits for the previous
// block's loads and LDS reads
__device__ __forceinline__ bool plan_next(const QPlan& p, int bin, int k, int& qb) {
  if (k >= p.ipb || p.blk[bin * p.ipb + k] == PLAN_NONE) return false;
  qb = p.blk[bin * p.ipb + k];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  return true;
}

// Persistent launches.  The hardware hands workgroups to the 8 XCDs round-robin
// and, inside an XCD, to its 4 shader engines round-robin, strictly in index
// order: a workgroup waits for a free CU in its own shader engine while other
// engines sit idle (timeline probes at n = 18432, 8 heads: 22 us of such gaps
// per CU in the 1.25 ms key-stationary launch), and the XCDs run at different
// speeds (5-8% apart), which no static assignment can follow.  With more blocks
// than CUs the grid is therefore one workgroup per CU, and blocks come from 8
// queues, one per XCD (workgroup w runs on XCD w % 8): queue x holds the blocks
// of the x-th eighth of the (b, h), bh in [x BH / 8, (x + 1) BH / 8), one
// (b, h) after the other, heaviest block first within each, so the XCD's CUs
// sweep the rows of one (b, h) together and share them in its L2.  A
// workgroup's first block is fixed by its index; after each block (the dK/dV
// kernel: shortly before) thread 0 takes the next entry of its own queue with
// one device-scope atomic add (about 1.2 us), and once that queue is drained,
// entries of the other queues, skipping those that a bit mask marks drained.  The last workgroup to find every queue drained
// returns the counters to zero, so each launch finds them cleared.  Which
// workgroup runs a block does not change its result: every block is computed
// whole by one workgroup.
struct WorkQ {
  // counters of this launch (nullptr = plain grid), a slot of WQ_STRIDE words:
  // [0, 8) queue heads, [8] mask of drained queues, [10, 12) the done word
  // (64-bit: workgroups finished in the low half, blocks they ran in the high
  // half), [12] fault flag (sticky: the launches never clear it)
  unsigned* ctr;
  int slots;  // workgroups per queue (grid / 8); their first blocks are not counted
};
constexpr int WQ_DRAINED = 8, WQ_DONE = 10, WQ_FAULT = 12, WQ_CLEAR = 12;

// Set (bit 0) by a persistent launch whose blocks did not add up to its block
// count, i.e. that found its counters not cleared at launch (lh_attn_status
// reads and resets it with the slots that flagged).
__device__ unsigned g_wq_fault;

// first (b, h) of queue x; queue x holds [wq_lo(x), wq_lo(x + 1))
__device__ __forceinline__ int wq_lo(int x, int BH) { return (int)(((long long)x * BH) >> 3); }
__device__ __forceinline__ int wq_len(int x, int nblk, int BH) { return (wq_lo(x + 1, BH) - wq_lo(x, BH)) * nblk; }

// (b, h) and block of entry j of queue x
__device__ __forceinline__ void wq_decode(int x, int j, int nblk, int BH, bool heavy_last, int& bh, int& blk) {
  const int i = j / nblk, r = j - i * nblk;
  bh = wq_lo(x, BH) + i;
  blk = heavy_last ? nblk - 1 - r : r;
}

// First block of this workgroup; false when it has none.
__device__ __forceinline__ bool wq_first(const WorkQ& q, int nblk, int BH, bool heavy_last, int& bh, int& blk) {
  if (!q.ctr) {
    schedule(blockIdx.x, nblk, BH, bh, blk, heavy_last);
    return true;
  }
  const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
  if (j >= wq_len(x, nblk, BH)) return false;
  wq_decode(x, j, nblk, BH, heavy_last, bh, blk);
  return true;
}

// The counter address as a per-lane (VGPR) value.  Every work-queue atomic is
// made by one lane, and with a per-lane address the compiler's atomic
// optimizer leaves it alone: for a uniform address it would read the result at
// once, or, for a value it cannot prove uniform, scan the active lanes in a
// loop that addresses lanes through M0 (which the direct loads' inline
// assembly assumes no compiler instruction touches).
__device__ __forceinline__ unsigned* lane_addr(unsigned* p) {
  int zero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
  return p + zero;
}
__device__ __forceinline__ unsigned long long* lane_addr64(unsigned* p) {
  return reinterpret_cast<unsigned long long*>(lane_addr(p));
}

// Thread 0, shortly before its workgroup's block ends: reserve the next entry
// of the workgroup's own queue.  Returns the counter's old value c (the entry
// is slots + c, valid while below the queue's length), or -1 when the queue has
// no counted entries; wq_next takes it as `reserved`.  Its first use is there,
// so the atomic's latency hides behind the rest of the block.  The address is
// made per-lane because the compiler's rewrite of a uniform-address atomic
// reads the result at once.
__device__ __forceinline__ int wq_reserve(const WorkQ& q, int nblk, int BH) {
  const int x = blockIdx.x & 7;
  if (wq_len(x, nblk, BH) <= q.slots) return -1;
  return (int)atomicAdd(lane_addr(q.ctr + x), 1u);
}

// Next block of this workgroup (persistent launches; false: none left), from
// thread 0's reservation (wq_reserve's value; -1: none made) or by taking
// entries itself.  Every thread calls it once the previous block's LDS reads
// are done, with nrun the number of blocks the workgroup has run; s is two
// ints of LDS.  The previous block's direct-to-LDS loads are waited for here.
//
// A workgroup that finds no block left adds itself and its block count to the
// done word.  The one that completes the workgroup count checks that the blocks
// add up to the launch's (nblk * BH; fewer when a queue head was not zero at
// launch, so entries were skipped) and returns the counters to zero.  A
// mismatch, or a workgroup count already past the grid, sets the slot's fault
// flag and g_wq_fault.  With the done word itself not zero at launch, an
// earlier workgroup believes it is the last and clears the counters while
// others still run; those then sweep the queues again, which repeats blocks
// (same arithmetic, same values) but skips none, and leave the slot not clear,
// which lh_attn_status finds once the device is idle.  A dirty drained mask
// only keeps other XCDs from entries that their owners still take.  No path
// waits on another workgroup, so a dirty slot cannot hang a launch.
__device__ __forceinline__ bool wq_next(const WorkQ& q, int nblk, int BH, bool heavy_last, int reserved, int nrun,
                                        int& bh, int& blk, int* s) {
  if (threadIdx.x == 0) {
    const int x0 = blockIdx.x & 7;
    int found = -1, fx = x0;
    unsigned drained = 0;
    int d = 0;
    if (reserved >= 0) {  // the own queue was asked already
      if (q.slots + reserved < wq_len(x0, nblk, BH))
        found = q.slots + reserved;
      else
        drained = atomicOr(lane_addr(q.ctr + WQ_DRAINED), 1u << x0);
      d = 1;
    }
    for (; d < 8 && found < 0; ++d) {
      const int x = (x0 + d) & 7;
      const int len = wq_len(x, nblk, BH);
      if (len <= q.slots || ((drained >> x) & 1)) {
        if (d == 0) drained = atomicOr(lane_addr(q.ctr + WQ_DRAINED), 0u);  // no counted entries here: learn which queues are drained
        continue;
      }
      const int j = q.slots + (int)atomicAdd(lane_addr(q.ctr + x), 1u);
      if (j < len) {
        found = j;
        fx = x;
      } else if (d == 0) {  // own queue drained: mark it, and learn which others are
        drained = atomicOr(lane_addr(q.ctr + WQ_DRAINED), 1u << x);
      } else {
        atomicOr(lane_addr(q.ctr + WQ_DRAINED), 1u << x);
      }
    }
    if (found < 0) {
      const unsigned long long old =
          atomicAdd(lane_addr64(q.ctr + WQ_DONE), 1ull | ((unsigned long long)(unsigned)nrun << 32));
      const unsigned wg = (unsigned)old;
      if (wg >= gridDim.x ||
          (wg == gridDim.x - 1 && (unsigned)(old >> 32) + (unsigned)nrun != (unsigned)nblk * (unsigned)BH)) {
        atomicOr(lane_addr(q.ctr + WQ_FAULT), 1u);
        atomicOr(lane_addr(&g_wq_fault), 1u);
      }
      if (wg == gridDim.x - 1) {
#pragma unroll
        for (int i = 0; i < WQ_CLEAR; ++i) atomicExch(lane_addr(q.ctr + i), 0u);
      }
    }
    s[0] = found;
    s[1] = fx;
  }
  __builtin_amdgcn_s_waitcnt(0);  // all of this wave's loads have landed
  __syncthreads();
  const int j = __builtin_amdgcn_readfirstlane(s[0]), x = __builtin_amdgcn_readfirstlane(s[1]);
  if (j < 0) return false;
  wq_decode(x, j, nblk, BH, heavy_last, bh, blk);
  return true;
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

// LDS byte address of a __shared__ pointer (wave-uniform)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)(p));
}

// Direct global->LDS loads: lane l writes its 16 (g2l16) or 4 (g2l4) bytes at
// lds_base + 16 l (4 l); lds_base is wave-uniform and goes through M0.  They
// are issued as inline assembly: the compiler's wait-count bookkeeping treats
// the builtin as a FLAT access that may also touch LDS and then turns every
// later LDS-read wait of the wave into lgkmcnt(0), which serialises the
// operand reads that feed the MFMAs.  Their completion is tracked by the
// vector-memory counter only; every caller waits for it explicitly (wait_vm,
// wait_loads) before a barrier publishes the data.  Loads the compiler does
// know about stay correctly waited: the counter completes in order, so an
// extra untracked load only makes the compiler's counts conservative.  M0 is
// a reserved register that the compiler may assume unchanged across inline
// assembly; no compiler-generated instruction of this file uses it (checked
// on the generated gfx950 assembly by tests/test_isa.py).
__device__ __forceinline__ void g2l16(const bf16_t* g, bf16_t* lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr(lds_base))
               : "memory", "m0");
}
__device__ __forceinline__ void g2l4(const void* g, void* lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_addr(lds_base))
               : "memory", "m0");
}

// wait until at most N vector-memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
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

// MFMA A operands read from a tile (the plain forms of lds_row / lds_tr below):
//   row operand of tile row r, k-slice c, lane half hh (d = 16c + 8hh .. +7):
//     the 16 bytes at element r * 128 + (((2c + hh) ^ swz(r)) << 3);
//   transposed operand of X^T, column d = 32 db + lane % 32, k-slots u = rows
//     r0 + 8 (u / 4) + 4 (lane / 32) + u % 4 (r0 a multiple of 16): within each
//     16-lane group, ds_read_b64_tr_b16 returns to lane i, element e, the 16-bit
//     word i % 4 of the 8 bytes addressed by lane i / 4 + 4e, so lane (g, j)
//     (g = lane / 16, j = lane % 16) reads row r = r0 + 4 (lane / 32) + j / 4,
//     chunk ch = 4 db + 2 (g & 1) + (j & 3) / 2, sub-word offset 4 (j & 1), and
//     the same at row r + 8 for the operand's upper half.

// Lane-constant parts of the operand addresses above, as byte offsets inside
// a 16 KB tile, arranged so that a k-slice / column block is folded in with
// one XOR:
//   row operand (r, c, hh)             at row ^ (c << 5), + 8192 for rows 32..63
//   transposed operand (r0, db) lo / hi at tr0 ^ (db << 6) and tr1 ^ (db << 6), + 256 r0
// (the chunk swizzle is an XOR, and 2c + hh = 2c ^ hh, 4 db + C = 4 db ^ C).
// Recomputing the few XORs per tile keeps the addresses out of long-lived registers.
struct LaneLds {
  uint32_t row, tr0, tr1;
};

__device__ __forceinline__ LaneLds lane_lds(int lane) {
  const int l32 = lane & 31, hh = lane >> 5, j = lane & 15, g = lane >> 4;
  const int rl = 4 * hh + (j >> 2), C = 2 * (g & 1) + ((j & 3) >> 1);
  LaneLds o;
  o.row = (uint32_t)(l32 * 256) | ((uint32_t)(swz(l32) ^ hh) << 4);
  o.tr0 = (uint32_t)(rl * 256) | ((uint32_t)(C ^ swz(rl)) << 4) | ((uint32_t)(j & 1) << 3);
  o.tr1 = (uint32_t)((rl + 8) * 256) | ((uint32_t)(C ^ swz(rl + 8)) << 4) | ((uint32_t)(j & 1) << 3);
  return o;
}

// row operand of tile rows 32 qb + lane%32, k-slice c
__device__ __forceinline__ u32x4 lds_row(const bf16_t* tile, const LaneLds& ll, int qb, int c) {
  return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(tile) + ((ll.row ^ ((uint32_t)c << 5)) +
                                                                                 8192u * qb));
}

// transposed operand of tile rows r0 .., column block db
__device__ __forceinline__ u32x4 lds_tr(const bf16_t* tile, const LaneLds& ll, int r0, int db) {
  const char* t = reinterpret_cast<const char*>(tile);
  const uint32_t x = (uint32_t)db << 6, o = 256u * r0;
  const u32x2 a = ld_tr16(reinterpret_cast<const bf16_t*>(t + ((ll.tr0 ^ x) + o)));
  const u32x2 b = ld_tr16(reinterpret_cast<const bf16_t*>(t + ((ll.tr1 ^ x) + o)));
  return u32x4{a.x, a.y, b.x, b.y};
}

// 8 fp32 accumulator values v = 8*c2 .. 8*c2+7 -> bf16 B operand
template <typename T>
__device__ __forceinline__ u32x4 pack_frag(const floatx16& s, int c2) {
  const int v = 8 * c2;
  return u32x4{cvt2<T>(s[v + 0], s[v + 1]), cvt2<T>(s[v + 2], s[v + 3]), cvt2<T>(s[v + 4], s[v + 5]), cvt2<T>(s[v + 6], s[v + 7])};
}

// key index held in accumulator slot v of a 32-key block
__device__ __forceinline__ int slot_key(int v, int hh) { return 8 * (v >> 2) + 4 * hh + (v & 3); }

template <typename T>
__device__ __forceinline__ void store_rows(bf16_t* row, const floatx16 (&acc)[4], float sc, int hh) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w.x = cvt2<T>(acc[d][4 * g + 0] * sc, acc[d][4 * g + 1] * sc);
      w.y = cvt2<T>(acc[d][4 * g + 2] * sc, acc[d][4 * g + 3] * sc);
      *reinterpret_cast<u32x2*>(row + d * 32 + 8 * g + 4 * hh) = w;
    }
  }
}

#define SCHED_GROUP(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
constexpr int SG_MFMA = 0x008, SG_DSR = 0x100;

// ===========================================================================
// forward (query-stationary)
// ===========================================================================
struct FwdState {
  floatx16 o[4];
  float m;  // running max in raw (unscaled) score units
  float l;  // this lane's half of the row sum
};

template <typename T>
__device__ __forceinline__ void fwd_tile(FwdState& st, const u32x4 (&qf)[8], const bf16_t* Ks, const bf16_t* Vs,
                                         int k0, int my_q, int n, int lane, float sl2, bool mask) {
  const int hh = lane >> 5;
  const LaneLds ll = lane_lds(lane);
  floatx16 s[2];
  {
    // operand i: key block i & 1, k-slice i >> 1, so consecutive MFMAs feed
    // different accumulators; each operand is read FWD_AHEAD MFMAs early
    u32x4 kf[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) kf[i] = lds_row(Ks, ll, i & 1, i >> 1);
    s[0] = mfma<T>(kf[0], qf[0], floatx16{});
    s[1] = mfma<T>(kf[1], qf[0], floatx16{});
#pragma unroll
    for (int i = 2; i < 16; ++i) s[i & 1] = mfma<T>(kf[i], qf[i >> 1], s[i & 1]);
    SCHED_GROUP(SG_DSR, FWD_AHEAD);
#pragma unroll
    for (int i = 0; i < 16 - FWD_AHEAD; ++i) {
      SCHED_GROUP(SG_DSR, 1);
      SCHED_GROUP(SG_MFMA, 1);
    }
    SCHED_GROUP(SG_MFMA, FWD_AHEAD);
  }
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
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int v = 0; v < 16; ++v) s[kb][v] = ex2(fmaf(s[kb][v], sl2, nm));
  }
  u32x4 pf[2][2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    pf[kb][0] = pack_frag<T>(s[kb], 0);
    pf[kb][1] = pack_frag<T>(s[kb], 1);
  }
  // Row sum of the bf16 P that the P V product uses, two terms per v_dot2
  // (16 instructions instead of 32 adds); the weights of O then sum to 1
  // exactly, up to the fp32 accumulation.
  {
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        ls = dot2one<T>(pf[kb][h].x, ls);
        ls = dot2one<T>(pf[kb][h].y, ls);
        ls = dot2one<T>(pf[kb][h].z, ls);
        ls = dot2one<T>(pf[kb][h].w, ls);
      }
    st.l += ls;
  }
  {
    // operand i: column block i & 3 (consecutive MFMAs feed different
    // accumulators), key rows 32 (i >> 3) + 16 ((i >> 2) & 1); two transposing
    // reads each, FWD_AHEAD operands ahead of their MFMAs
    u32x4 vf[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) vf[i] = lds_tr(Vs, ll, (i >> 3) * 32 + 16 * ((i >> 2) & 1), i & 3);
#pragma unroll
    for (int i = 0; i < 16; ++i) st.o[i & 3] = mfma<T>(vf[i], pf[i >> 3][(i >> 2) & 1], st.o[i & 3]);
    SCHED_GROUP(SG_DSR, 2 * FWD_AHEAD);
#pragma unroll
    for (int i = 0; i < 16 - FWD_AHEAD; ++i) {
      SCHED_GROUP(SG_DSR, 2);
      SCHED_GROUP(SG_MFMA, 1);
    }
    SCHED_GROUP(SG_MFMA, FWD_AHEAD);
  }
}

// One query block qb of (b, h) bh.
template <typename T, int EPI>  // 0: O + LSE;  1: rounded row norms of O into `scores`
__device__ __forceinline__ void fwd_block(const AttnArgs& a, int bh, int qb, bf16_t* K0, bf16_t* K1, bf16_t* V0,
                                          bf16_t* V1) {
  constexpr int BM = 32 * QW;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
    if (j < nt && k0 <= qw + 31) fwd_tile<T>(st, qf, Ks, Vs, k0, my_q, n, lane, a.sl2, j >= nfull);
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
    store_rows<T>(a.out + ((int64_t)bh * n + my_q) * LH_D, st.o, inv_l, hh);
    if (hh == 0) a.lse[(int64_t)bh * n + my_q] = l > 0.f ? st.m * a.sl2 + __log2f(l) : -INFINITY;
  } else {
    float ss = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const uint32_t w = cvt2<T>(st.o[d][v] * inv_l, st.o[d][v + 1] * inv_l);
        const float x0 = T::lo(w), x1 = T::hi(w);
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
      a.scores[((int64_t)b * a.Ho + ho) * a.S_tot + t] = round_to<T>(sqrtf(ss));
    }
  }
}

template <typename T, int EPI>
__global__ __launch_bounds__(64 * QW, 8 / QW) void attn_fwd_kernel(const AttnArgs a, const QPlan p, const WorkQ q) {
  __shared__ __attribute__((aligned(1024))) bf16_t K0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t K1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V1[TILE];
  __shared__ int wq_s[2];
  int bh, qb, bin = 0;
  bool have;
  if (p.bph) {
    plan_first(p, bh, bin, qb);
    have = qb != PLAN_NONE;
  } else {
    have = wq_first(q, a.nq, a.BH, true, bh, qb);
    if (!have && q.ctr) have = wq_next(q, a.nq, a.BH, true, -1, 0, bh, qb, wq_s);
  }
  for (int k = 1; have; ++k) {
    fwd_block<T, EPI>(a, bh, qb, K0, K1, V0, V1);
    // the next block starts after this one's last tile reads
    if (p.bph)
      have = plan_next(p, bin, k, qb);
    else
      have = q.ctr && wq_next(q, a.nq, a.BH, true, -1, k, bh, qb, wq_s);
  }
}

// ===========================================================================
// backward dQ (query-stationary)
// ===========================================================================
template <typename T, bool CTR>
__device__ __forceinline__ void dq_tile(floatx16 (&acc)[4], float& rsum, const u32x4 (&qf)[8], const u32x4 (&df)[8],
                                        const bf16_t* Ks, const bf16_t* Vs, int k0, int my_q, int n, int lane,
                                        float sl2, float nlse, float dlt, bool mask) {
  const int hh = lane >> 5;
  const LaneLds ll = lane_lds(lane);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    floatx16 s, dp;
    __builtin_amdgcn_s_setprio(1);
    {
      // operand i: k-slice i >> 1 of K (i even, for S) or V (i odd, for dP), so
      // consecutive MFMAs feed the two accumulators; reads run DQ_AHEAD ahead
      u32x4 f[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) f[i] = lds_row((i & 1) ? Vs : Ks, ll, kb, i >> 1);
      floatx16 dinit;
#pragma unroll
      for (int v = 0; v < 16; ++v) dinit[v] = -dlt;  // the accumulator ends as dP - delta
      s = mfma<T>(f[0], qf[0], floatx16{});
      dp = mfma<T>(f[1], df[0], dinit);
#pragma unroll
      for (int i = 2; i < 16; i += 2) {
        s = mfma<T>(f[i], qf[i >> 1], s);
        dp = mfma<T>(f[i + 1], df[i >> 1], dp);
      }
      SCHED_GROUP(SG_DSR, DQ_AHEAD);
#pragma unroll
      for (int i = 0; i < 16 - DQ_AHEAD; ++i) {
        SCHED_GROUP(SG_DSR, 1);
        SCHED_GROUP(SG_MFMA, 1);
      }
      SCHED_GROUP(SG_MFMA, DQ_AHEAD);
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
    for (int v = 0; v < 16; ++v) s[v] = ex2(fmaf(s[v], sl2, nlse)) * dp[v];
    const u32x4 f0 = pack_frag<T>(s, 0), f1 = pack_frag<T>(s, 1);
    if (CTR) {
      // this lane's share of the row sum of the bf16 dS that the product below
      // uses (two independent chains)
      float r0 = dot2one<T>(f0.x, 0.f);
      float r1 = dot2one<T>(f1.x, 0.f);
      r0 = dot2one<T>(f0.y, r0);
      r1 = dot2one<T>(f1.y, r1);
      r0 = dot2one<T>(f0.z, r0);
      r1 = dot2one<T>(f1.z, r1);
      r0 = dot2one<T>(f0.w, r0);
      r1 = dot2one<T>(f1.w, r1);
      rsum += r0 + r1;
    }
    __builtin_amdgcn_s_setprio(1);
    {
      // operand i: column block i & 3, key rows kb * 32 + 16 (i >> 2)
      u32x4 g[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = lds_tr(Ks, ll, kb * 32 + 16 * (i >> 2), i & 3);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i & 3] = mfma<T>(g[i], (i >> 2) ? f1 : f0, acc[i & 3]);
      SCHED_GROUP(SG_DSR, 2 * DQ_AHEAD2);
#pragma unroll
      for (int i = 0; i < 8 - DQ_AHEAD2; ++i) {
        SCHED_GROUP(SG_DSR, 2);
        SCHED_GROUP(SG_MFMA, 1);
      }
      SCHED_GROUP(SG_MFMA, DQ_AHEAD2);
    }
    __builtin_amdgcn_s_setprio(0);
  }
}

// dQ of one query block qb of (b, h) bh.
//
// Key centring.  dQ_i = scale sum_t dS_it k_t, and sum_t dS_it = 0 on every
// row (dS = P (dP - delta), delta = sum_t P dP), so dQ_i = scale sum_t dS_it
// (k_t - c) for any vector c.  The product takes dS rounded to bf16, whose
// errors (and those of delta, formed from the bf16 O) multiply k_t: with a
// large component that the keys share (a channel constant over the keys, as
// trained models' keys often have), that product alone errs far beyond the
// bf16 tolerance.  The kernel therefore also sums r_i = sum_t bf16(dS_it) (the
// same bf16 values, by v_dot2 against ones) and subtracts scale r_i c at the
// end, which gives scale sum_t bf16(dS_it) (k_t - c): the rounding errors then
// multiply k_t - c instead of k_t.  c is the fp32 mean of 64 key rows spread
// evenly over the block's causal key range, read with plain loads beside the
// first tile's direct loads (kc: 128 + 8 x 129 floats of LDS).
//
// The row sum costs 16 VALU instructions per tile, which the VALU-bound loop
// feels (+2.9% at cfg2), and it changes the result only where the keys share
// a component: the errors it removes scale with |c|, those left with
// |k_t - c|.  A block therefore applies it only when |c|^2 > E|k - c|^2 / 16
// over the sample (|c| above a quarter of the keys' spread about it); N(0, 1)
// keys (|c|^2 about 2 against 126) skip it and give the uncentred result.
// Every wave forms the same sums in the same order, so the choice is uniform.
template <typename T>
__device__ __forceinline__ void dq_block(const AttnArgs& a, int bh, int qb, bf16_t* K0, bf16_t* K1, bf16_t* V0,
                                         bf16_t* V1, float* kc) {
  constexpr int BM = 32 * QW;
  int tid = threadIdx.x;  // opaque, as in dkdv_block
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = a.n;
  const BhRows m = bh_rows(a, bh);
  const int q0 = qb * BM, qw = q0 + wave * 32, my_q = qw + l32;
  const int qc = min(my_q, n - 1);

  u32x4 qf[8], df[8];
  {
    bool pooled;
    const uint32_t o = row_off(m, my_q, pooled) + 8 * hh;
    const bf16_t* p = (pooled ? m.qp : m.q) + o;
    // formed from opaque copies so that the compiler does not hoist per-lane
    // address parts out of the persistent block loop (they would spill)
    int row = qc, half = hh;
    asm volatile("" : "+v"(row), "+v"(half));
    const bf16_t* pd = a.dout + ((int64_t)bh * n + row) * LH_D + 8 * half;
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
  // key sample for the centre: thread t reads 16 bytes (dims 8 (t % 16) ..) of
  // sample rows t / 16 and t / 16 + 32, sample s at key (s kend) / 64
  u32x4 ks0, ks1;
  {
    const int ch = tid & 15, s0 = tid >> 4;
    bool pooled;
    uint32_t o = row_off(m, (s0 * kend) >> 6, pooled);
    ks0 = ldg16((pooled ? m.kp : m.k) + o + 8 * ch);
    o = row_off(m, ((s0 + 32) * kend) >> 6, pooled);
    ks1 = ldg16((pooled ? m.kp : m.k) + o + 8 * ch);
  }
  wait_loads();
  float* kcp = kc + 128;  // per wave: 128 dim sums, then the sum of squares
  int ln = lane;  // opaque: its LDS addresses are not hoisted out of the block loop (they would spill)
  asm volatile("" : "+v"(ln));
  {
    // sum the two rows, then over the four lanes of this wave that hold the
    // same 8 dims, then over the waves in LDS; beside it the sum of squares
    float c8[8], k2 = 0.f;
    const uint32_t w0[4] = {ks0.x, ks0.y, ks0.z, ks0.w}, w1[4] = {ks1.x, ks1.y, ks1.z, ks1.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = T::lo(w0[e]), a1 = T::hi(w0[e]);
      const float b0 = T::lo(w1[e]), b1 = T::hi(w1[e]);
      c8[2 * e] = a0 + b0;
      c8[2 * e + 1] = a1 + b1;
      k2 = fmaf(a0, a0, fmaf(a1, a1, fmaf(b0, b0, fmaf(b1, b1, k2))));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      c8[e] += __shfl_xor(c8[e], 16);
      c8[e] += __shfl_xor(c8[e], 32);
    }
#pragma unroll
    for (int x = 1; x < 64; x <<= 1) k2 += __shfl_xor(k2, x);
    if (ln < 16) {
      float4* dst = reinterpret_cast<float4*>(kcp + wave * 132 + 8 * ln);
      dst[0] = float4{c8[0], c8[1], c8[2], c8[3]};
      dst[1] = float4{c8[4], c8[5], c8[6], c8[7]};
    }
    if (ln == 0) kcp[wave * 132 + 128] = k2;
  }
  __syncthreads();
  bool ctr;
  {
    // every wave: lane l forms dims 2l, 2l+1 of the centre, the wave |c|^2,
    // and all waves the same E|k|^2 (the same additions in the same order)
    float ca = 0.f, cb = 0.f, kk = 0.f;
#pragma unroll
    for (int w = 0; w < QW; ++w) {
      const float2 v = *reinterpret_cast<const float2*>(kcp + w * 132 + 2 * ln);
      ca += v.x;
      cb += v.y;
      kk += kcp[w * 132 + 128];
    }
    ca *= 1.0f / 64.0f;
    cb *= 1.0f / 64.0f;
    float cc = fmaf(ca, ca, cb * cb);
#pragma unroll
    for (int x = 1; x < 64; x <<= 1) cc += __shfl_xor(cc, x);
    // E|k - c|^2 = E|k|^2 - |c|^2 over the sample: centre when |c|^2 > that / 16
    ctr = __builtin_amdgcn_readfirstlane((int)(17.0f * cc > kk * (1.0f / 64.0f)));
    if (wave == 0) *reinterpret_cast<float2*>(kc + 2 * ln) = float2{ca, cb};  // read in the epilogue
  }

  floatx16 acc[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) acc[d] = floatx16{};
  float rsum = 0.f;
  const int nfull = min((qw + 1) / BN, n / BN);

  auto step = [&](auto C, int j, const bf16_t* Ks, const bf16_t* Vs, bf16_t* Kn, bf16_t* Vn) {
    const int k0 = j * BN;
    if (j + 1 < nt) issue_rows<QW>(Kn, m.k, m.kp, Vn, m.v, m.vp, m, rr, wave, lane);
    if (j + 2 < nt) load_rows<QW>(rr, m, k0 + 2 * BN, wave, lane);
    if (j < nt && k0 <= qw + 31)
      dq_tile<T, decltype(C)::value>(acc, rsum, qf, df, Ks, Vs, k0, my_q, n, lane, a.sl2, nlse, dlt, j >= nfull);
    wait_loads();
    __syncthreads();
  };
  if (ctr) {
    for (int j = 0; j < nt; j += 2) {
      step(std::true_type{}, j, K0, V0, K1, V1);
      step(std::true_type{}, j + 1, K1, V1, K0, V0);
    }
  } else {
    for (int j = 0; j < nt; j += 2) {
      step(std::false_type{}, j, K0, V0, K1, V1);
      step(std::false_type{}, j + 1, K1, V1, K0, V0);
    }
  }

  // the two lane halves hold the two halves of each row's keys
  rsum += __shfl_xor(rsum, 32);
  if (my_q >= n) return;
  // acc[d][4 g + e] is dim 32 d + 8 g + 4 hh + e
  if (ctr)
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 c = *reinterpret_cast<const float4*>(kc + 32 * d + 8 * g + 4 * hh);
      acc[d][4 * g + 0] = fmaf(-rsum, c.x, acc[d][4 * g + 0]);
      acc[d][4 * g + 1] = fmaf(-rsum, c.y, acc[d][4 * g + 1]);
      acc[d][4 * g + 2] = fmaf(-rsum, c.z, acc[d][4 * g + 2]);
      acc[d][4 * g + 3] = fmaf(-rsum, c.w, acc[d][4 * g + 3]);
    }
  {
    int row = my_q, half = hh;
    asm volatile("" : "+v"(row), "+v"(half));
    store_rows<T>(a.dq + ((int64_t)bh * n + row) * LH_D, acc, a.scale, half);
  }
}

template <typename T>
__global__ __launch_bounds__(64 * QW, 8 / QW) void attn_bwd_dq_kernel(const AttnArgs a, const QPlan p, const WorkQ q) {
  __shared__ __attribute__((aligned(1024))) bf16_t K0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t K1[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V0[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t V1[TILE];
  __shared__ __attribute__((aligned(16))) float KC[128 + QW * 132];  // key centre + per-wave partial sums
  __shared__ int wq_s[2];
  int bh, qb, bin = 0;
  bool have;
  if (p.bph) {
    plan_first(p, bh, bin, qb);
    have = qb != PLAN_NONE;
  } else {
    have = wq_first(q, a.nq, a.BH, true, bh, qb);
    if (!have && q.ctr) have = wq_next(q, a.nq, a.BH, true, -1, 0, bh, qb, wq_s);
  }
  for (int k = 1; have; ++k) {
    dq_block<T>(a, bh, qb, K0, K1, V0, V1, KC);
    // the next block starts after this one's last tile reads
    if (p.bph)
      have = plan_next(p, bin, k, qb);
    else
      have = q.ctr && wq_next(q, a.nq, a.BH, true, -1, k, bh, qb, wq_s);
  }
}

// ===========================================================================
// backward dK, dV (key-stationary, two roles in ping-pong)
//
// A block owns 128 keys: 4 wave pairs of 32 keys, the two waves of a pair on
// one SIMD.  Wave 0-3 of a pair ("P wave") holds K and accumulates dV: in its
// MFMA phase it forms S = Q K^T of the current 64-query tile and adds
// P^T dO of the previous one; in its VALU phase it turns S into P and hands P
// (bf16) to its partner through LDS.  Wave 4-7 ("dS wave") holds V and
// accumulates dK: dP = dO V^T of the current tile and dS^T Q of the previous
// one; in its VALU phase dS = P (dP - delta).  The dS waves run one phase
// behind, and a block barrier closes every phase, so on each SIMD one wave
// feeds the matrix core while the other runs its VALU work, and each wave needs
// only half of the key-side registers.  The S and dP accumulators start from
// -lse / (scale log2 e) and delta of their query (the dS waves hold -V, so
// their accumulator ends as delta - dP): the VALU phases read nothing from LDS
// but the exchanged P, because reads issued there would queue behind the
// partner waves' operand reads.  Q/dO tiles (+ lse, delta) rotate through 4
// LDS buffers, filled by direct loads that the VALU phases issue (the P waves
// the Q tiles, the dS waves the dO tiles).  Deterministic: no atomics.
// ===========================================================================
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Tile copies of the key-stationary kernel: direct global->LDS loads, each wave
// 16 rows of a 64-row tile (four 1 KB loads, row 16 w + 4 i + lane / 16 in
// load i), plus at most one 64-entry row of 4-byte values.
__device__ __forceinline__ void copy_q16(bf16_t* qt, const BhRows& m, const int (&r)[4], int w, int lane) {
  const int rsub = lane >> 4, slot = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * w + 4 * i + rsub;
    const bool pooled = r[i] >= m.split;
    const uint32_t rel = (uint32_t)(r[i] - (pooled ? m.split : 0));
    g2l16((pooled ? m.qp : m.q) + rel * (uint32_t)(pooled ? m.ps : m.ss) + 8 * (slot ^ swz(row)),
          qt + (16 * w + 4 * i) * LH_D);
  }
}

__device__ __forceinline__ void copy_d16(bf16_t* dt, const bf16_t* dbase, int row0, int n, int w, int lane) {
  const int rsub = lane >> 4, slot = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * w + 4 * i + rsub;
    g2l16(dbase + (uint32_t)min(row0 + row, n - 1) * LH_D + 8 * (slot ^ swz(row)), dt + (16 * w + 4 * i) * LH_D);
  }
}

// Selected-row indices of the rows wave w copies in a 64-row tile at row0
// (clamped to the last row), read from global memory.
template <bool GATHER>
__device__ __forceinline__ void rows16(int (&r)[4], const BhRows& m, int row0, int w, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = min(row0 + 16 * w + 4 * i + (lane >> 4), m.last);
    r[i] = GATHER ? m.idx[s] : s;
  }
}

// The same indices from a tile's 64 entries staged in LDS.
__device__ __forceinline__ void rows16_lds(int (&r)[4], const int* ix, int w, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = ix[16 * w + 4 * i + (lane >> 4)];
}

// Issue order of an MFMA phase built as: the NINIT accumulator-start reads,
// 16 transposing reads (8 operands), 16 more, their 8 + 8 MFMAs, 8 + 8 row
// reads, their 8 + 8 MFMAs.  Each operand group is read while the previous
// group's MFMAs run, so LDS latency overlaps the matrix core and at most two
// operand groups are live.
template <int NINIT>
__device__ __forceinline__ void mma_phase_order() {
  SCHED_GROUP(SG_DSR, NINIT + 16);  // the accumulator-start reads, then the first 8 operands
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    SCHED_GROUP(SG_DSR, 2);
    SCHED_GROUP(SG_MFMA, 1);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    SCHED_GROUP(SG_DSR, 1);
    SCHED_GROUP(SG_MFMA, 1);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    SCHED_GROUP(SG_DSR, 1);
    SCHED_GROUP(SG_MFMA, 1);
  }
  SCHED_GROUP(SG_MFMA, 8);
}

// S accumulator start of a 32-query block for the P waves: slot 4 g + i of
// lane (hh, j) holds query 8 g + 4 hh + i (g, i < 4) and starts from
// lse[query] * nisl2.  Each lane reads one float4 (group g = lane % 4), and
// quad broadcasts (DPP quad_perm [g, g, g, g], fused into the multiply) give it
// the other three groups: 1 KB of LDS reads per wave instead of 4 KB of float4s
// that the 32 lanes of a half share.  (The dS waves keep the plain reads: their
// start values need no multiply, and 32 separate DPP moves cost more than the
// reads they save.)
template <int G>
__device__ __forceinline__ float quad_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), G * 0x55, 0xF, 0xF, false));
}

__device__ __forceinline__ void s_start(floatx16& a, const float* lse, float nisl2) {
  const int lane = __lane_id();
  const float4 x = *reinterpret_cast<const float4*>(lse + 8 * (lane & 3) + 4 * (lane >> 5));
#define LH_QB(G)                            \
  a[4 * G + 0] = quad_bcast<G>(x.x) * nisl2; \
  a[4 * G + 1] = quad_bcast<G>(x.y) * nisl2; \
  a[4 * G + 2] = quad_bcast<G>(x.z) * nisl2; \
  a[4 * G + 3] = quad_bcast<G>(x.w) * nisl2;
  LH_QB(0) LH_QB(1) LH_QB(2) LH_QB(3)
#undef LH_QB
}

// MFMA phase of a P wave: dV += dO^T P of the previous tile (Dp, pp), then
// S of the current tile (Qc).  Operands are read a group ahead of their MFMAs.
template <typename T>
__device__ __forceinline__ void pw_mma(floatx16 (&s)[2], floatx16 (&dva)[4], const u32x4 (&kf)[8],
                                       const u32x4 (&pp)[2][2], const bf16_t* Qc, const bf16_t* Dp,
                                       const LaneLds& ll, const float* lse, float nisl2) {
  // S starts from -lse / (scale log2 e) of its query, so that P = exp2(S scale log2 e)
  floatx16 si[2];
  s_start(si[0], lse, nisl2);
  s_start(si[1], lse + 32, nisl2);
  u32x4 oa[8], ob[8], ka[8], kb[8];
  // operand i: rows 32 qb + 16 c2 with qb = i & 1, c2 = (i >> 1) & 1; column block db = i >> 2 (+2)
#pragma unroll
  for (int i = 0; i < 8; ++i) oa[i] = lds_tr(Dp, ll, 32 * (i & 1) + 16 * ((i >> 1) & 1), i >> 2);
#pragma unroll
  for (int i = 0; i < 8; ++i) ob[i] = lds_tr(Dp, ll, 32 * (i & 1) + 16 * ((i >> 1) & 1), 2 + (i >> 2));
#pragma unroll
  for (int i = 0; i < 8; ++i) dva[i >> 2] = mfma<T>(oa[i], pp[i & 1][(i >> 1) & 1], dva[i >> 2]);
#pragma unroll
  for (int c = 0; c < 8; ++c) ka[c] = lds_row(Qc, ll, 0, c);
#pragma unroll
  for (int i = 0; i < 8; ++i) dva[2 + (i >> 2)] = mfma<T>(ob[i], pp[i & 1][(i >> 1) & 1], dva[2 + (i >> 2)]);
#pragma unroll
  for (int c = 0; c < 8; ++c) kb[c] = lds_row(Qc, ll, 1, c);
  s[0] = mfma<T>(ka[0], kf[0], si[0]);
#pragma unroll
  for (int c = 1; c < 8; ++c) s[0] = mfma<T>(ka[c], kf[c], s[0]);
  s[1] = mfma<T>(kb[0], kf[0], si[1]);
#pragma unroll
  for (int c = 1; c < 8; ++c) s[1] = mfma<T>(kb[c], kf[c], s[1]);

  mma_phase_order<2>();
}

// MFMA phase of a dS wave: dK += Q^T dS of the previous tile (Qp, dsf), then
// dP of the current tile (Dc).
template <typename T>
__device__ __forceinline__ void dw_mma(floatx16 (&dp)[2], floatx16 (&dka)[4], const u32x4 (&vf)[8],
                                       const u32x4 (&dsf)[2][2], const bf16_t* Dc, const bf16_t* Qp,
                                       const LaneLds& ll, const float* delta) {
  // vf holds -V, and the accumulator starts from delta of its query: it ends as delta - dP
  floatx16 di[2];
  {
    const int hh = __lane_id() >> 5;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 d4 = *reinterpret_cast<const float4*>(delta + qb * 32 + 8 * g + 4 * hh);
        di[qb][4 * g + 0] = d4.x;
        di[qb][4 * g + 1] = d4.y;
        di[qb][4 * g + 2] = d4.z;
        di[qb][4 * g + 3] = d4.w;
      }
  }
  u32x4 oa[8], ob[8], ka[8], kb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) oa[i] = lds_tr(Qp, ll, 32 * (i & 1) + 16 * ((i >> 1) & 1), i >> 2);
#pragma unroll
  for (int i = 0; i < 8; ++i) ob[i] = lds_tr(Qp, ll, 32 * (i & 1) + 16 * ((i >> 1) & 1), 2 + (i >> 2));
#pragma unroll
  for (int i = 0; i < 8; ++i) dka[i >> 2] = mfma<T>(oa[i], dsf[i & 1][(i >> 1) & 1], dka[i >> 2]);
#pragma unroll
  for (int c = 0; c < 8; ++c) ka[c] = lds_row(Dc, ll, 0, c);
#pragma unroll
  for (int i = 0; i < 8; ++i) dka[2 + (i >> 2)] = mfma<T>(ob[i], dsf[i & 1][(i >> 1) & 1], dka[2 + (i >> 2)]);
#pragma unroll
  for (int c = 0; c < 8; ++c) kb[c] = lds_row(Dc, ll, 1, c);
  dp[0] = mfma<T>(ka[0], vf[0], di[0]);
#pragma unroll
  for (int c = 1; c < 8; ++c) dp[0] = mfma<T>(ka[c], vf[c], dp[0]);
  dp[1] = mfma<T>(kb[0], vf[0], di[1]);
#pragma unroll
  for (int c = 1; c < 8; ++c) dp[1] = mfma<T>(kb[c], vf[c], dp[1]);

  mma_phase_order<8>();
}

// LDS of the key-stationary block (dkdv_block): Q and dO tiles, their lse and
// delta, the P hand-over and the staged Q row indices.
struct DkdvLds {
  bf16_t *Q0, *Q1, *Q2, *Q3, *D0, *D1, *D2, *D3;
  float *L0, *L1, *L2, *L3;
  u32x4 (*EX)[4][64];
  int (*IX)[BN];
};

// dK, dV of key block kblk of (b, h) bh (128 keys).  q and nblk name the
// work queue (entries per (b, h)) that thread 0 reserves its next entry from,
// shortly before the block ends; returns that reservation (-1: none).
template <typename T, bool GATHER>
__device__ __forceinline__ int dkdv_block(const AttnArgs& a, const WorkQ& q, int nblk, int bh, int kblk,
                                          const DkdvLds& lds) {
  bf16_t *Q0 = lds.Q0, *Q1 = lds.Q1, *Q2 = lds.Q2, *Q3 = lds.Q3;
  bf16_t *D0 = lds.D0, *D1 = lds.D1, *D2 = lds.D2, *D3 = lds.D3;
  float *L0 = lds.L0, *L1 = lds.L1, *L2 = lds.L2, *L3 = lds.L3;
  u32x4(*EX)[4][64] = lds.EX;
  int(*IX)[BN] = lds.IX;
  // the thread index as an opaque value: values derived from it are formed here,
  // per block, not hoisted out of a persistent block loop (they would stay live
  // through the other blocks' code and spill)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, pair = wave & 3;
  const LaneLds ll = lane_lds(lane);
  // wave-uniform by construction; said explicitly, or the compiler keeps bh * n (and the
  // addresses derived from it) in vector registers and spills them across the loop
  bh = __builtin_amdgcn_readfirstlane(bh);
  kblk = __builtin_amdgcn_readfirstlane(kblk);
  const int n = a.n;
  const BhRows m = bh_rows(a, bh);
  const int k0 = kblk * BMK, kw = k0 + 32 * pair, my_k = kw + l32;

  u32x4 kf[8];  // K (P wave) or -V (dS wave) rows of this lane's key
  {
    bool pooled;
    const uint32_t o = row_off(m, my_k, pooled) + 8 * hh;
    const bf16_t* p = grp ? (pooled ? m.vp : m.v) + o : (pooled ? m.kp : m.k) + o;
#pragma unroll
    for (int c = 0; c < 8; ++c) kf[c] = ldg16(p + 16 * c);
    if (grp) {  // the dS waves hold -V (bf16 sign flips are exact)
#pragma unroll
      for (int c = 0; c < 8; ++c) kf[c] ^= 0x80008000u;
    }
  }
  const int64_t bhn = (int64_t)bh * n;
  const bf16_t* dbase = a.dout + bhn * LH_D;
  const float* lse_row = a.lse_in + bhn;
  const float* dlt_row = a.delta + bhn;
  const int jt0 = k0 / BN;  // first query tile that sees these keys
  const int nt = (n + BN - 1) / BN;

  // Copies.  The P waves copy the Q tiles (+ lse on wave 0, the Q row indices
  // of a later tile on wave 1), the dS waves the dO tiles (+ delta on wave 4),
  // each wave 16 rows, in their VALU phases: in step j the P waves copy tile
  // j + 2 (phase 2j + 1) and the dS waves tile j + 3 (phase 2j + 2), each into
  // the buffer last read in phase 2j - 1 (Q, lse) or 2j (dO, delta); every
  // wave waits for its previous step's copies before the barrier closing its
  // VALU phase, so tile t is in LDS from phase 2t on (Q) or 2t + 1 on (dO).
  // Here: Q tiles jt0, jt0 + 1, dO tiles jt0 .. jt0 + 2, and the indices of
  // Q tiles jt0 + 2, jt0 + 3.
  if (grp == 0) {
    int r[4];
    rows16<GATHER>(r, m, jt0 * BN, pair, lane);
    copy_q16(Q0, m, r, pair, lane);
    rows16<GATHER>(r, m, (jt0 + 1) * BN, pair, lane);
    copy_q16(Q1, m, r, pair, lane);
    if (pair == 0) {
      g2l4(lse_row + min(jt0 * BN + lane, n - 1), L0);
      g2l4(lse_row + min((jt0 + 1) * BN + lane, n - 1), L1);
    }
    if (GATHER && pair == 1) {
      g2l4(m.idx + min((jt0 + 2) * BN + lane, m.last), IX[2]);
      g2l4(m.idx + min((jt0 + 3) * BN + lane, m.last), IX[3]);
    }
  } else {
    copy_d16(D0, dbase, jt0 * BN, n, pair, lane);
    copy_d16(D1, dbase, (jt0 + 1) * BN, n, pair, lane);
    copy_d16(D2, dbase, (jt0 + 2) * BN, n, pair, lane);
    if (pair == 0) {
      g2l4(dlt_row + min(jt0 * BN + lane, n - 1), L0 + BN);
      g2l4(dlt_row + min((jt0 + 1) * BN + lane, n - 1), L1 + BN);
      g2l4(dlt_row + min((jt0 + 2) * BN + lane, n - 1), L2 + BN);
    }
  }
  // the first step's dV / dK terms multiply zeros with buffer 3: make it finite
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    reinterpret_cast<u32x4*>(Q3)[tid + 512 * i] = u32x4{};
    reinterpret_cast<u32x4*>(D3)[tid + 512 * i] = u32x4{};
  }
  wait_loads();  // the first tiles and the zeros are in LDS
  block_barrier();

  floatx16 acc[4];  // dV (P wave) or dK (dS wave)
#pragma unroll
  for (int d = 0; d < 4; ++d) acc[d] = floatx16{};
  floatx16 sc[2] = {floatx16{}, floatx16{}};  // S - lse/(scale log2 e) (P wave) or delta - dP (dS wave)
  u32x4 op[2][2] = {{u32x4{}, u32x4{}}, {u32x4{}, u32x4{}}};  // P or dS, bf16 operands
  const float sl2 = a.sl2, nisl2 = -1.0f / a.sl2;

  // Step j: MFMA phase (tile j, and the previous tile's accumulation), then the
  // VALU phase with this step's copies.  The step count is rounded up to a
  // multiple of 4 so that the buffers rotate statically; steps past the last
  // tile copy clamped rows.  Each role runs its own loop (same barrier count)
  // and is register-allocated on its own.
  auto pstep = [&](int j, const bf16_t* Qc, const float* Lc, const bf16_t* Dp, bf16_t* Qn, float* Ln,
                   const int* ixc, int* ixn) {
    if (j <= nt) {  // steps past nt (the rounding to 4) would multiply masked tiles and add zeros
      __builtin_amdgcn_s_setprio(1);
      pw_mma<T>(sc, acc, kf, op, Qc, Dp, ll, Lc, nisl2);
      __builtin_amdgcn_s_setprio(0);
    }
    block_barrier();
    {  // copy Q tile j + 2 (indices staged two steps ago), its lse, and the indices of tile j + 4
      int r[4];
      if (GATHER)
        rows16_lds(r, ixc, pair, lane);
      else
        rows16<false>(r, m, (j + 2) * BN, pair, lane);
      copy_q16(Qn, m, r, pair, lane);
      if (pair == 0) g2l4(lse_row + min((j + 2) * BN + lane, n - 1), Ln);
      if (GATHER && pair == 1) g2l4(m.idx + min((j + 4) * BN + lane, m.last), ixn);
    }
    if (j < nt) {  // P = exp2(S sl2 - lse), masked causally and past n
      const int q0t = j * BN;
      const bool mask = q0t < kw + 31 || q0t + BN > n;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        if (mask) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int q = q0t + qb * 32 + slot_key(v, hh);
            if (my_k > q || q >= n) sc[qb][v] = -INFINITY;
          }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) sc[qb][v] = ex2(sc[qb][v] * sl2);
        op[qb][0] = pack_frag<T>(sc[qb], 0);
        op[qb][1] = pack_frag<T>(sc[qb], 1);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) EX[pair][i][lane] = op[i >> 1][i & 1];
    } else {  // past the last tile the accumulation steps add zeros
      op[0][0] = op[0][1] = op[1][0] = op[1][1] = u32x4{};
    }
    // all but this step's copies have landed
    if (pair == 0 || (GATHER && pair == 1))
      wait_vm<5>();
    else
      wait_vm<4>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this phase's LDS writes have landed
    block_barrier();
  };
  auto dstep = [&](int j, const bf16_t* Dc, const float* Lc, const bf16_t* Qp, bf16_t* Dn, float* Ln) {
    if (j <= nt) {
      __builtin_amdgcn_s_setprio(1);
      dw_mma<T>(sc, acc, kf, op, Dc, Qp, ll, Lc + BN);
      __builtin_amdgcn_s_setprio(0);
    }
    block_barrier();
    copy_d16(Dn, dbase, (j + 3) * BN, n, pair, lane);  // dO tile j + 3 and its delta
    if (pair == 0) g2l4(dlt_row + min((j + 3) * BN + lane, n - 1), Ln + BN);
    if (j < nt) {  // dS = P (dP - delta), P from the partner P wave
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const u32x4 e0 = EX[pair][2 * qb][lane], e1 = EX[pair][2 * qb + 1][lane];
        float pv[16];
        unpack8_t<T>(uint4{e0.x, e0.y, e0.z, e0.w}, pv);
        unpack8_t<T>(uint4{e1.x, e1.y, e1.z, e1.w}, pv + 8);
#pragma unroll
        for (int v = 0; v < 16; ++v) sc[qb][v] = pv[v] * -sc[qb][v];  // P (dP - delta)
        op[qb][0] = pack_frag<T>(sc[qb], 0);
        op[qb][1] = pack_frag<T>(sc[qb], 1);
      }
    } else {
      op[0][0] = op[0][1] = op[1][0] = op[1][1] = u32x4{};
    }
    if (pair == 0)
      wait_vm<5>();
    else
      wait_vm<4>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the partner's P was read
    block_barrier();
  };
  int next = -1;  // thread 0: the reserved next entry
  if (grp == 0) {
    for (int j = jt0; j <= nt; j += 4) {
      pstep(j, Q0, L0, D3, Q2, L2, IX[2], IX[0]);
      pstep(j + 1, Q1, L1, D0, Q3, L3, IX[3], IX[1]);
      pstep(j + 2, Q2, L2, D1, Q0, L0, IX[0], IX[2]);
      pstep(j + 3, Q3, L3, D2, Q1, L1, IX[1], IX[3]);
    }
    // the dS waves' last phase is still to run: reserve the next block now
    if (q.ctr && threadIdx.x == 0) next = wq_reserve(q, nblk, a.BH);
    block_barrier();
  } else {
    block_barrier();  // the dS waves run one phase behind
    for (int j = jt0; j <= nt; j += 4) {
      dstep(j, D0, L0, Q3, D3, L3);
      dstep(j + 1, D1, L1, Q0, D0, L0);
      dstep(j + 2, D2, L2, Q1, D1, L1);
      dstep(j + 3, D3, L3, Q2, D2, L2);
    }
  }
  if (my_k < n) {
    // the row addresses are formed here, not held through the loops (they would spill)
    int row = my_k, half = hh;
    asm volatile("" : "+v"(row), "+v"(half));
    if (grp == 0)
      store_rows<T>(a.dv + ((int64_t)bh * n + row) * LH_D, acc, 1.0f, half);
    else
      store_rows<T>(a.dk + ((int64_t)bh * n + row) * LH_D, acc, a.scale, half);
  }
  return next;
}

template <typename T, bool GATHER>
__global__ __launch_bounds__(512, 1) void attn_bwd_dkdv_kernel(const AttnArgs a, const WorkQ q) {
  __shared__ __attribute__((aligned(1024))) bf16_t Q0[TILE], Q1[TILE], Q2[TILE], Q3[TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t D0[TILE], D1[TILE], D2[TILE], D3[TILE];
  __shared__ __attribute__((aligned(16))) float L0[2 * BN], L1[2 * BN], L2[2 * BN], L3[2 * BN];  // lse, delta
  __shared__ u32x4 EX[4][4][64];  // P handed from each P wave to its dS wave
  __shared__ __attribute__((aligned(16))) int IX[4][BN];  // selected-row indices of the Q tiles to copy
  __shared__ int wq_s[2];
  const DkdvLds lds{Q0, Q1, Q2, Q3, D0, D1, D2, D3, L0, L1, L2, L3, EX, IX};
  int bh, kblk;
  bool have = wq_first(q, a.nq, a.BH, false, bh, kblk);  // early key blocks see the most queries
  if (!have && q.ctr) have = wq_next(q, a.nq, a.BH, false, -1, 0, bh, kblk, wq_s);
  int nrun = 0;  // blocks this workgroup has run
  while (have) {
    // wave-uniform by construction; said explicitly, or the compiler keeps bh * n (and the
    // addresses derived from it) in vector registers and spills them across the loop
    bh = __builtin_amdgcn_readfirstlane(bh);
    kblk = __builtin_amdgcn_readfirstlane(kblk);
    const int next = dkdv_block<T, GATHER>(a, q, a.nq, bh, kblk, lds);
    if (!q.ctr) break;
    have = wq_next(q, a.nq, a.BH, false, next, ++nrun, bh, kblk, wq_s);  // the previous block's copies are waited for there
  }
}

// ===========================================================================
// GLA scorer: simple gated linear attention over the dilated virtual heads,
//   o_t = scale * sum_{s <= t} exp(G_t - G_s) (q_t . k_s) v_s,  G = cumsum(g),
// and the L2 norm of o_t rounded to the row type (bf16 or fp16), itself
// rounded to that type, as the base score.
// Chunked form (chunks of 64 tokens, processed in order): with b the
// chunk-local inclusive cumsum of g and H the state after the previous chunk,
//   o = scale * ((Q K^T) o exp(b_t - b_s), causal) V + scale * exp(b_t) Q H
//   H <- exp(b_last) H + (K o exp(b_last - b_s))^T V.
// The sequence of each (b, virtual head, direction) is cut into P segments of
// whole chunks so that P times more workgroups share the chip.  A first pass
// (gla_state_kernel, P - 1 segments) runs only the state recurrence of each
// segment from a zero state and stores its final state dH_s and its decay
// D_s = prod exp(b_last) in a workspace; the scoring pass of segment s starts
// from H = sum_{s' < s} (prod_{s' < s'' < s} D_s'') dH_s', formed by the
// recurrence H <- D_s' H + dH_s', and walks its own chunks.  P = 1 is the plain
// sequential walk.
// One workgroup (8 waves) owns one segment of one (b, virtual head,
// direction).  The state is kept transposed, H^T [j][i] (j: value dim, i: key
// dim), in fp32 MFMA accumulators (wave w: rows 32 (w >> 1), columns 64 (w & 1)
// .. + 63) with a copy rounded to the row type in LDS as the operand of the
// inter-chunk product (fp16 rows: fp16 MFMAs, an fp16 state copy).
// As in the forward kernel, products come out transposed (A^T, O^T), so an
// accumulator column is a token.  Per chunk: phase 1 (waves 0-2) forms the
// three causal 32x32 blocks of A^T and hands them over in LDS as packed
// operands, wave 3 the decay factors; phase 2 every wave forms one 32-token x
// 32-column block of O^T (norm partials to LDS) and updates its state blocks;
// phase 3 writes the new state copy and wave 7 finishes the norms.  Tiles
// of the next chunk are loaded (direct global->LDS) during the current one.
// ===========================================================================
struct GlaArgs {
  const bf16_t *q, *k, *v;  // [B, S, H, D] contiguous
  const float* g;           // [B, S, H] fp32 log gates
  float *sqk, *skq;         // [B, H, S_tot]: base level written
  float* ws;                // P > 1: segment states [units][P - 1][8 waves][2][16][64], then decays [units][P - 1]
  int B, S, H, dil, T, S_tot;
  int P, cps;               // segments per sequence, chunks per segment
  float scale;
};

constexpr int GLA_WS_WAVE = 2 * 16 * 64;  // fp32 state values held by one wave
constexpr int GLA_WS_SEG = 8 * GLA_WS_WAVE;

__device__ __forceinline__ void gla_issue(bf16_t* tile, const bf16_t* base, uint32_t stride, int t0, int last,
                                          int w, int lane) {
  const int rsub = lane >> 4, slot = lane & 15;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 8 * w + 4 * i + rsub;
    const int t = min(t0 + r, last);
    g2l16(base + (uint32_t)t * stride + 8 * (slot ^ swz(r)), tile + (8 * w + 4 * i) * LH_D);
  }
}

// bf16 element (row, col) of a swizzled 64 x 128 tile
__device__ __forceinline__ int tile_elem(int row, int col) { return row * LH_D + ((((col >> 3) ^ swz(row)) << 3) | (col & 7)); }

// The (b, virtual head, direction) sequence and segment of a workgroup:
// logical block (seq * nseg + seg) * 2 + dir, taken through xcd_block so that
// the two directions of a segment, which stream the same q, k and v rows in
// step, run on one XCD and share its L2.
struct GlaSeq {
  const bf16_t *qb, *kb, *vb;
  const float* gb;
  float* scores;
  uint32_t stride;
  int unit, seg, VH;
};

__device__ __forceinline__ GlaSeq gla_seq(const GlaArgs& a, int nseg) {
  GlaSeq s;
  s.VH = a.dil * a.H;
  const int blk = (int)xcd_block(blockIdx.x, gridDim.x);
  const int dir = blk & 1;
  const int rest = blk >> 1;
  const int seq = rest / nseg;
  s.seg = rest - seq * nseg;
  s.unit = seq * 2 + dir;
  const int b = seq / s.VH, vh = seq % s.VH;
  const int r = vh / a.H, ho = vh % a.H;
  s.stride = (uint32_t)s.VH * LH_D;  // elements between consecutive tokens of a virtual head
  const int64_t off = (int64_t)b * a.S * a.H * LH_D + (int64_t)vh * LH_D;
  s.qb = (dir ? a.k : a.q) + off;
  s.kb = (dir ? a.q : a.k) + off;
  s.vb = a.v + off;
  s.gb = a.g + (int64_t)b * a.S * a.H + vh;
  s.scores = (dir ? a.skq : a.sqk) + ((int64_t)b * a.H + ho) * a.S_tot + r;
  return s;
}

template <int CTRL>
__device__ __forceinline__ float dpp0(float x) {  // DPP move, 0 where the source lane is outside the row
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// Chunk-local inclusive cumsum of g in log2 units (tokens past the end add 0):
// Hillis-Steele within each 16-lane row by DPP row shifts, then the row totals
// carried across rows.
__device__ __forceinline__ float gla_cumsum(const float* G, int nvalid, int lane) {
  float x = (lane < nvalid) ? G[lane] * 1.4426950408889634f : 0.f;
  x += dpp0<0x111>(x);  // row_shr:1
  x += dpp0<0x112>(x);  // row_shr:2
  x += dpp0<0x114>(x);  // row_shr:4
  x += dpp0<0x118>(x);  // row_shr:8
  const float r0 = lane_value(x, 15), r1 = lane_value(x, 31), r2 = lane_value(x, 47);
  const int row = lane >> 4;
  const float r01 = r0 + r1;
  return x + (row == 0 ? 0.f : row == 1 ? r0 : row == 2 ? r01 : r01 + r2);
}

__device__ __forceinline__ void gla_decays(float x, int nvalid, int lane, float* Es, float* Fs) {
  const float bl = lane_value(x, nvalid - 1);
  Es[lane] = ex2(x);
  Fs[lane] = lane < nvalid ? ex2(bl - x) : 0.f;
}

// H^T <- exp(b_last) H^T + (V o f)^T K for this wave's two state blocks
template <typename T>
__device__ __forceinline__ void gla_state_update(floatx16 (&hs)[2], float el, const bf16_t* Vt, const bf16_t* Kt,
                                                 const float* Fs, const LaneLds& ll, int sjb, int sib, int hh) {
#pragma unroll
  for (int q = 0; q < 2; ++q) hs[q] *= el;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    u32x4 vt = lds_tr(Vt, ll, 16 * kk, sjb);
    const float4 f0 = *reinterpret_cast<const float4*>(&Fs[16 * kk + 4 * hh]);
    const float4 f1 = *reinterpret_cast<const float4*>(&Fs[16 * kk + 8 + 4 * hh]);
    const float fv[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = T::lo(vt[e]) * fv[2 * e];
      const float hi = T::hi(vt[e]) * fv[2 * e + 1];
      vt[e] = cvt2<T>(lo, hi);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) hs[q] = mfma<T>(vt, lds_tr(Kt, ll, 16 * kk, sib + q), hs[q]);
  }
}

// Copy of this wave's state blocks, rounded to the element type, into the LDS operand H^T
template <typename T>
__device__ __forceinline__ void gla_state_copy(bf16_t (*HT)[TILE], const floatx16 (&hs)[2], int sjb, int sib,
                                               int l32, int hh) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int i = 32 * (sib + q) + l32;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int j = 32 * sjb + slot_key(v, hh);
      HT[j >> 6][tile_elem(j & 63, i)] = (bf16_t)(cvt2<T>(hs[q][v], 0.f) & 0xffffu);
    }
  }
}

// State pass (E: the row element type): segment s < P - 1 of a sequence,
// from a zero state, K / V / g tiles only; stores the final fp32 state blocks
// and the segment's decay.
// Every wave forms the chunk's decay factors itself (in a wave-private LDS
// row), so one barrier per chunk (tile reuse) suffices.
template <typename E>
__global__ __launch_bounds__(512, 1) void gla_state_kernel(const GlaArgs a) {
  __shared__ __attribute__((aligned(1024))) bf16_t Kt[2][TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t Vt[2][TILE];
  __shared__ __attribute__((aligned(16))) float Gs[2][64];
  __shared__ __attribute__((aligned(16))) float Fw[8][64];  // wave w's exp(b_last - b_s)
  const int tid = threadIdx.x, lane = tid & 63, hh = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const LaneLds ll = lane_lds(lane);
  const GlaSeq sq = gla_seq(a, a.P - 1);
  const int T = a.T, last = T - 1;
  const int nch = (T + 63) / 64;
  const int c0 = sq.seg * a.cps, c1 = min(nch, c0 + a.cps);
  const int sjb = w >> 1, sib = 2 * (w & 1);
  floatx16 hs[2] = {floatx16{}, floatx16{}};
  float dec = 1.f;

  auto issue = [&](int c, int buf) {
    const int t0 = 64 * c;
    gla_issue(Kt[buf], sq.kb, sq.stride, t0, last, w, lane);
    gla_issue(Vt[buf], sq.vb, sq.stride, t0, last, w, lane);
    if (w == 0) g2l4(sq.gb + (int64_t)min(t0 + lane, last) * sq.VH, Gs[buf]);
  };
  issue(c0, 0);
  wait_loads();
  __syncthreads();
  for (int c = c0; c < c1; ++c) {
    const int buf = (c - c0) & 1;
    const int nvalid = min(64, T - 64 * c);
    if (c + 1 < c1) issue(c + 1, buf ^ 1);
    const float x = gla_cumsum(Gs[buf], nvalid, lane);
    const float bl = lane_value(x, nvalid - 1);
    Fw[w][lane] = lane < nvalid ? ex2(bl - x) : 0.f;
    const float el = ex2(bl);
    dec *= el;
    gla_state_update<E>(hs, el, Vt[buf], Kt[buf], Fw[w], ll, sjb, sib, hh);
    wait_loads();
    __syncthreads();
  }
  float* out = a.ws + ((int64_t)(sq.unit * (a.P - 1) + sq.seg) * 8 + w) * GLA_WS_WAVE + lane;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int v = 0; v < 16; ++v) out[(q * 16 + v) * 64] = hs[q][v];
  }
  if (tid == 0) {
    const int64_t units = (int64_t)a.B * sq.VH * 2;
    a.ws[units * (a.P - 1) * GLA_WS_SEG + sq.unit * (a.P - 1) + sq.seg] = dec;
  }
}

// Scoring pass.  Per chunk c two phases, each closed by a barrier:
//   A: every wave forms its O^T block (inter-chunk H^T Q^T + intra-chunk
//      V^T A^T), its norm partials, and updates its state blocks;
//   B: the new bf16 state copy; wave 7 finishes chunk c's norms; waves 0-2
//      form the A^T blocks of chunk c + 1 and wave 3 its decay factors (both
//      double-buffered), so that phase A of the next chunk starts at once.
// Tiles of chunk c + 2 are issued at the start of phase B of chunk c, into the
// buffers chunk c has just released, and waited for at the end of phase A of
// chunk c + 1.
template <typename E>
__global__ __launch_bounds__(512, 1) void gla_scores_kernel(const GlaArgs a) {
  __shared__ __attribute__((aligned(1024))) bf16_t Qt[2][TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t Kt[2][TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t Vt[2][TILE];
  __shared__ __attribute__((aligned(1024))) bf16_t HT[2][TILE];  // bf16 H^T: rows j, columns i
  __shared__ __attribute__((aligned(16))) float Gs[2][64];
  __shared__ __attribute__((aligned(16))) float Es[2][64], Fs[2][64];  // exp(b_t), exp(b_last - b_s) (0 past the end)
  __shared__ __attribute__((aligned(16))) float Bw[3][64];             // b of waves 0-2 (wave-private rows)
  __shared__ u32x4 AP[2][3][2][64];  // packed A^T blocks (s0,t0), (s0,t1), (s1,t1) per buffer
  __shared__ float RED[4][64];       // norm partials per column block
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const LaneLds ll = lane_lds(lane);
  const GlaSeq sq = gla_seq(a, a.P);
  const int T = a.T, last = T - 1;
  const int nch = (T + 63) / 64;
  const int c0 = sq.seg * a.cps, c1 = min(nch, c0 + a.cps);

  const int sjb = w >> 1, sib = 2 * (w & 1);  // state blocks (j block, i blocks sib, sib + 1)
  const int otb = w & 1, odb = w >> 1;         // output block (token block, column block)
  floatx16 hs[2] = {floatx16{}, floatx16{}};
  if (sq.seg > 0) {
    // state entering the segment from the earlier segments' states and decays
    const int64_t units = (int64_t)a.B * sq.VH * 2;
    const float* dec = a.ws + units * (a.P - 1) * GLA_WS_SEG + (int64_t)sq.unit * (a.P - 1);
    for (int s = 0; s < sq.seg; ++s) {
      const float d = dec[s];
      const float* in = a.ws + ((int64_t)(sq.unit * (a.P - 1) + s) * 8 + w) * GLA_WS_WAVE + lane;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int v = 0; v < 16; ++v) hs[q][v] = fmaf(d, hs[q][v], in[(q * 16 + v) * 64]);
      }
    }
  }
  gla_state_copy<E>(HT, hs, sjb, sib, l32, hh);

  auto issue = [&](int c, int buf) {
    const int t0 = 64 * c;
    gla_issue(Qt[buf], sq.qb, sq.stride, t0, last, w, lane);
    gla_issue(Kt[buf], sq.kb, sq.stride, t0, last, w, lane);
    gla_issue(Vt[buf], sq.vb, sq.stride, t0, last, w, lane);
    if (w == 0) g2l4(sq.gb + (int64_t)min(t0 + lane, last) * sq.VH, Gs[buf]);
  };
  // A^T blocks (waves 0-2) and decay factors (wave 3) of chunk c from buffer buf
  auto prep = [&](int c, int buf) {
    if (w >= 4) return;
    const int nvalid = min(64, T - 64 * c);
    const float x = gla_cumsum(Gs[buf], nvalid, lane);
    if (w == 3) {
      gla_decays(x, nvalid, lane, Es[buf], Fs[buf]);
      return;
    }
    Bw[w][lane] = x;  // read back below by this wave only (LDS keeps a wave's order)
    const int tb = w == 0 ? 0 : 1, sbk = w == 2 ? 1 : 0;
    floatx16 acc = floatx16{};
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) acc = mfma<E>(lds_row(Kt[buf], ll, sbk, cc), lds_row(Qt[buf], ll, tb, cc), acc);
    const int t = 32 * tb + l32;
    const float bt = Bw[w][t];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int s0 = 32 * sbk + 8 * g + 4 * hh;  // slots v = 4 g .. 4 g + 3 hold keys s0 .. s0 + 3
      const float4 bs = *reinterpret_cast<const float4*>(&Bw[w][s0]);
      const float b4[4] = {bs.x, bs.y, bs.z, bs.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int v = 4 * g + r, s = s0 + r;
        acc[v] = (s <= t && s < nvalid) ? acc[v] * a.scale * ex2(bt - b4[r]) : 0.f;
      }
    }
    AP[buf][w][0][lane] = pack_frag<E>(acc, 0);
    AP[buf][w][1][lane] = pack_frag<E>(acc, 1);
  };

  issue(c0, 0);
  wait_loads();
  __syncthreads();
  if (c0 + 1 < c1) issue(c0 + 1, 1);
  prep(c0, 0);
  __syncthreads();

  for (int c = c0; c < c1; ++c) {
    const int buf = (c - c0) & 1;
    const int nvalid = min(64, T - 64 * c);
    // ---- phase A: O^T block (otb, odb), norm partials, state update
    {
      floatx16 oi = floatx16{}, oa = floatx16{};
      // inter-chunk: H^T rows of column block odb against the chunk's queries
#pragma unroll
      for (int cc = 0; cc < 8; ++cc)
        oi = mfma<E>(lds_row(HT[odb >> 1], ll, odb & 1, cc), lds_row(Qt[buf], ll, otb, cc), oi);
      // intra-chunk: V^T against the packed A^T blocks of this token block
#pragma unroll
      for (int sbk = 0; sbk < 2; ++sbk) {
        if (sbk > otb) break;
        const int blk = otb == 0 ? 0 : 1 + sbk;
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
          oa = mfma<E>(lds_tr(Vt[buf], ll, 32 * sbk + 16 * c2, odb), AP[buf][blk][c2][lane], oa);
      }
      const float et = Es[buf][32 * otb + l32] * a.scale;
      float ss = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float o = fmaf(oi[v], et, oa[v]);
        const float ob = round_to<E>(o);  // the output value as stored in the row type
        ss = fmaf(ob, ob, ss);
      }
      ss += __shfl_xor(ss, 32);
      if (hh == 0) RED[odb][32 * otb + l32] = ss;
      gla_state_update<E>(hs, Es[buf][nvalid - 1], Vt[buf], Kt[buf], Fs[buf], ll, sjb, sib, hh);
    }
    wait_loads();  // tiles of chunk c + 1
    __syncthreads();
    // ---- phase B: rounded copy of the new state; norms of chunk c; A^T and decays of chunk c + 1
    if (c + 2 < c1) issue(c + 2, buf);
    gla_state_copy<E>(HT, hs, sjb, sib, l32, hh);
    if (w == 7 && lane < nvalid) {
      const float ss = (RED[0][lane] + RED[1][lane]) + (RED[2][lane] + RED[3][lane]);
      sq.scores[(int64_t)(64 * c + lane) * a.dil] = round_to<E>(sqrtf(ss));
    }
    if (c + 1 < c1) prep(c + 1, buf ^ 1);
    __syncthreads();
  }
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

// CUs of the current device (cached per device); 0 when unknown.
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = -1;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c > 0 ? c : 0;
}

// Best-fit-decreasing packing of costs w into at most nb bins of capacity cap:
// each block, heaviest first, goes to the fullest bin it still fits in.
bool pack_bfd(const std::vector<int>& w, const std::vector<int>& order, int nb, long long cap,
              std::vector<std::vector<int>>& bins) {
  bins.assign(nb, {});
  std::vector<long long> load(nb, 0);
  int used = 0;
  for (int b : order) {
    int best = -1;
    for (int j = 0; j < used; ++j)
      if (load[j] + w[b] <= cap && (best < 0 || load[j] > load[best])) best = j;
    if (best < 0) {
      if (used == nb) return false;
      best = used++;
    }
    bins[best].push_back(b);
    load[best] += w[b];
  }
  return true;
}

// Query-block plan of a query-stationary launch over BH (b, h) of length n:
// bph = CUs / BH bins per (b, h), each (b, h)'s bins on one XCD.  A block of
// 32 QW queries costs its key tiles (counted in half tiles) plus about 1.5
// tiles of set-up and stores; the blocks are packed best-fit-decreasing into
// bph bins of the smallest capacity (binary search from the larger of the
// heaviest block and the mean) for which they fit.  No plan (one block per
// workgroup) when the bins would not fill whole XCDs or every block has a CU
// of its own anyway.  Plans are cached per geometry.  Returns the grid size.
std::atomic<int> g_schedule{0};  // LH_SCHED_* flags (lh_attn_set_schedule)

int make_plan(int BH, int n, QPlan& p) {
  p.bph = 0;
  p.ipb = 0;
  const int nb = (n + 32 * QW - 1) / (32 * QW);
  const int plain = nb * BH;
  if (g_schedule.load(std::memory_order_relaxed) & LH_SCHED_NO_PLAN) return plain;
  const int cus = cu_count();
  if (cus <= 0 || cus % 8 || BH % 8 || BH > cus || (cus / 8) % (BH / 8)) return plain;
  const int bph = cus / BH;
  if (nb <= bph || 2 * nb > 7 * bph || nb >= (int)PLAN_NONE) return plain;
  const long long key = ((long long)cus << 48) | ((long long)BH << 32) | (long long)n;
  static std::mutex mu;
  static std::map<long long, QPlan> cache;
  {
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
      p = it->second;
      return p.bph ? p.bph * BH : plain;
    }
  }
  std::vector<int> w(nb), order(nb);
  long long total = 0;
  for (int b = 0; b < nb; ++b) {
    w[b] = 2 * ((std::min((b + 1) * 32 * QW, n) + BN - 1) / BN) + 3;
    order[b] = b;
    total += w[b];
  }
  std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return w[x] > w[y]; });
  std::vector<std::vector<int>> bins, best;
  long long lo = std::max<long long>(w[order[0]], (total + bph - 1) / bph), hi = total;
  while (lo < hi) {  // smallest capacity the packing fits in (it always fits at the total)
    const long long mid = (lo + hi) / 2;
    if (pack_bfd(w, order, bph, mid, bins)) {
      best = bins;
      hi = mid;
    } else {
      lo = mid + 1;
    }
  }
  if (best.empty() || !pack_bfd(w, order, bph, lo, best)) pack_bfd(w, order, bph, total, best);
  int ipb = 0;
  for (auto& bn : best) ipb = std::max(ipb, (int)bn.size());
  if ((long long)ipb * bph <= QPLAN_MAX) {
    for (int j = 0; j < bph; ++j) {
      std::stable_sort(best[j].begin(), best[j].end(), [&](int x, int y) { return w[x] > w[y]; });
      for (int k = 0; k < ipb; ++k) p.blk[j * ipb + k] = k < (int)best[j].size() ? (uint16_t)best[j][k] : PLAN_NONE;
    }
    p.bph = bph;
    p.ipb = ipb;
  }
  std::lock_guard<std::mutex> g(mu);
  if (cache.size() >= 256) cache.clear();
  cache[key] = p;
  return p.bph ? p.bph * BH : plain;
}

// Work-queue counters of the persistent launches: one 128-byte slot per
// (device, stream), so launches that may run at the same time (different
// streams) never share counters, while launches on one stream run one after
// the other and each leaves its slot cleared.  A launch made while its stream
// is being captured into a graph gets a slot of its own that no other launch
// uses (graphs captured one after the other on one stream can be replayed on
// different streams at once; only a graph replayed beside itself races).  Past
// WQ_SLOTS slots on a device, launches fall back to the plain grid.
constexpr int WQ_SLOTS = 1024, WQ_STRIDE = 32;
__device__ __attribute__((aligned(256))) unsigned g_wq[WQ_SLOTS * WQ_STRIDE];

struct WqDevice {
  unsigned* base = nullptr;  // device address of g_wq (hipGetSymbolAddress)
  unsigned* fault = nullptr;  // device address of g_wq_fault
  int used = 0;
};

std::mutex& wq_mutex() {
  static std::mutex mu;
  return mu;
}

// the current device's slot array (caller holds wq_mutex); nullptr when unavailable
WqDevice* wq_device(int& dev) {
  static WqDevice devs[64];
  dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  WqDevice& d = devs[dev];
  if (!d.base) {
    void* ptr = nullptr;
    void* fptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_wq)) != hipSuccess || !ptr) return nullptr;
    if (hipGetSymbolAddress(&fptr, HIP_SYMBOL(g_wq_fault)) != hipSuccess || !fptr) return nullptr;
    d.base = static_cast<unsigned*>(ptr);
    d.fault = static_cast<unsigned*>(fptr);
  }
  return &d;
}

unsigned* wq_counters(hipStream_t st) {
  std::lock_guard<std::mutex> g(wq_mutex());
  int dev = 0;
  WqDevice* d = wq_device(dev);
  if (!d) return nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) return nullptr;
  if (cs != hipStreamCaptureStatusNone) {  // a captured launch: a slot of its own
    if (d->used == WQ_SLOTS) return nullptr;
    return d->base + (d->used++) * WQ_STRIDE;
  }
  static std::map<std::pair<int, std::pair<uintptr_t, std::thread::id>>, int> slot;
  // hipStreamPerThread names a different stream on every host thread
  const std::thread::id tid = st == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
  const auto key = std::make_pair(dev, std::make_pair(reinterpret_cast<uintptr_t>(st), tid));
  auto it = slot.find(key);
  if (it != slot.end()) return d->base + it->second * WQ_STRIDE;
  if (d->used == WQ_SLOTS) return nullptr;
  slot[key] = d->used;
  return d->base + (d->used++) * WQ_STRIDE;
}

// Grid of a launch over BH (b, h) of nblk blocks each: one workgroup per CU
// with work queues when there are 1 to 12 blocks per CU, else one block per
// workgroup.  Past 12 the plain grid's gaps and tail are a small share, and the
// kernels are power-limited, so CUs kept busier run at a lower clock: the
// dilated scorer at cfg4 (16 blocks per CU) measured 1% slower with queues.
int wq_grid(int nblk, int BH, hipStream_t st, WorkQ& q) {
  q.ctr = nullptr;
  q.slots = 0;
  const long long total = (long long)nblk * BH;
  const int cus = cu_count();
  if (cus <= 0 || cus % 8 || total <= cus || total > 12LL * cus) return (int)total;
  if (g_schedule.load(std::memory_order_relaxed) & LH_SCHED_NO_QUEUE) return (int)total;
  unsigned* c = wq_counters(st);
  if (!c) return (int)total;
  q.ctr = c;
  q.slots = cus / 8;
  return cus;
}

// Grid of a query-stationary launch: a packed plan where one applies, else as wq_grid.
int query_grid(int BH, int n, hipStream_t st, QPlan& p, WorkQ& q) {
  const int grid = make_plan(BH, n, p);
  q.ctr = nullptr;
  q.slots = 0;
  return p.bph ? grid : wq_grid((n + 32 * QW - 1) / (32 * QW), BH, st, q);
}

}  // namespace

extern "C" int lh_attn_fwd(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                           const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                           int split, const int32_t* indices, int B, int H, int n, int D, float scale, void* out,
                           float* lse, int dtype, void* stream) {
  AttnArgs a{};
  int rc = fill_rows(a, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale);
  if (rc) return rc;
  if (!out || !lse || !al16(out) || !valid_dtype(dtype)) return LH_ERR_INVALID_ARG;
  a.out = (bf16_t*)out; a.lse = lse;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  QPlan p;
  WorkQ wq;
  const int grid = query_grid(a.BH, a.n, st, p, wq);
  LH_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((attn_fwd_kernel<T, 0>), dim3(grid), dim3(64 * QW), 0, st, a, p, wq));
  LH_CHECK_LAUNCH();
  return LH_OK;
}

namespace {
// parts: bit 0 = dK/dV kernel, bit 1 = dQ kernel
int attn_bwd_parts(int parts, const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                   const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph, int split,
                   const int32_t* indices, int B, int H, int n, int D, float scale, const void* dout,
                   const float* lse, const float* delta, void* dq, void* dk, void* dv, int dtype, void* stream) {
  AttnArgs a{};
  int rc = fill_rows(a, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale);
  if (rc) return rc;
  if (!dout || !lse || !delta || !al16(dout) || !valid_dtype(dtype)) return LH_ERR_INVALID_ARG;
  if (indices && n < 8) return LH_ERR_UNSUPPORTED;  // gathered rows are indexed 8 at a time
  if ((parts & 1) && (!dk || !dv || !al16(dk) || !al16(dv))) return LH_ERR_INVALID_ARG;
  if ((parts & 2) && (!dq || !al16(dq))) return LH_ERR_INVALID_ARG;
  a.dout = (const bf16_t*)dout; a.lse_in = lse; a.delta = delta;
  a.dq = (bf16_t*)dq; a.dk = (bf16_t*)dk; a.dv = (bf16_t*)dv;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (parts & 1) {
    AttnArgs ak = a;
    ak.nq = (a.n + BMK - 1) / BMK;
    WorkQ wq;
    const int grid = wq_grid(ak.nq, ak.BH, st, wq);
    LH_DISPATCH_DTYPE(dtype, if (indices) hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, true>), dim3(grid), dim3(512),
                                                             0, st, ak, wq);
                      else hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, false>), dim3(grid), dim3(512), 0, st, ak,
                                              wq));
    LH_CHECK_LAUNCH();
  }
  if (parts & 2) {
    QPlan p;
    WorkQ wq;
    const int grid = query_grid(a.BH, a.n, st, p, wq);
    LH_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL(attn_bwd_dq_kernel<T>, dim3(grid), dim3(64 * QW), 0, st, a, p, wq));
    LH_CHECK_LAUNCH();
  }
  return LH_OK;
}
}  // namespace

extern "C" int lh_attn_bwd(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                           const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                           int split, const int32_t* indices, int B, int H, int n, int D, float scale,
                           const void* dout, const float* lse, const float* delta, void* dq, void* dk, void* dv,
                           int dtype, void* stream) {
  return attn_bwd_parts(3, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale, dout,
                        lse, delta, dq, dk, dv, dtype, stream);
}

extern "C" int lh_attn_bwd_dkdv(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                                const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                                int split, const int32_t* indices, int B, int H, int n, int D, float scale,
                                const void* dout, const float* lse, const float* delta, void* dk, void* dv,
                                int dtype, void* stream) {
  return attn_bwd_parts(1, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale, dout,
                        lse, delta, nullptr, dk, dv, dtype, stream);
}

extern "C" int lh_attn_bwd_dq(const void* q, const void* k, const void* v, int64_t sb, int64_t ss, int64_t sh,
                              const void* qp, const void* kp, const void* vp, int64_t pb, int64_t ps, int64_t ph,
                              int split, const int32_t* indices, int B, int H, int n, int D, float scale,
                              const void* dout, const float* lse, const float* delta, void* dq, int dtype,
                              void* stream) {
  return attn_bwd_parts(2, q, k, v, sb, ss, sh, qp, kp, vp, pb, ps, ph, split, indices, B, H, n, D, scale, dout,
                        lse, delta, dq, nullptr, nullptr, dtype, stream);
}

extern "C" int lh_attn_status(int* faults) {
  if (!faults) return LH_ERR_INVALID_ARG;
  *faults = 0;
  std::lock_guard<std::mutex> g(wq_mutex());
  int dev = 0;
  WqDevice* d = wq_device(dev);
  if (!d) return LH_ERR_RUNTIME;
  // With the device idle no launch is in flight, so every slot's counters must
  // be zero: a slot is faulty when a launch flagged it or when it is not clear.
  if (hipDeviceSynchronize() != hipSuccess) return LH_ERR_RUNTIME;
  std::vector<unsigned> w((size_t)WQ_SLOTS * WQ_STRIDE);
  if (hipMemcpy(w.data(), d->base, w.size() * sizeof(unsigned), hipMemcpyDeviceToHost) != hipSuccess)
    return LH_ERR_RUNTIME;
  unsigned flag = 0;
  if (hipMemcpy(&flag, d->fault, sizeof(flag), hipMemcpyDeviceToHost) != hipSuccess) return LH_ERR_RUNTIME;
  int n = 0;
  for (int i = 0; i < WQ_SLOTS; ++i) {
    unsigned* c = w.data() + (size_t)i * WQ_STRIDE;
    if (std::all_of(c, c + WQ_STRIDE, [](unsigned x) { return x == 0u; })) continue;
    ++n;
    std::fill(c, c + WQ_STRIDE, 0u);
    if (hipMemcpy(d->base + (size_t)i * WQ_STRIDE, c, WQ_STRIDE * sizeof(unsigned), hipMemcpyHostToDevice) !=
        hipSuccess)
      return LH_ERR_RUNTIME;
  }
  if (flag) {
    flag = 0;
    if (hipMemcpy(d->fault, &flag, sizeof(flag), hipMemcpyHostToDevice) != hipSuccess) return LH_ERR_RUNTIME;
    if (!n) n = 1;
  }
  *faults = n;
  return LH_OK;
}

extern "C" int lh_attn_set_schedule(int flags, int* previous) {
  if (flags & ~(LH_SCHED_NO_PLAN | LH_SCHED_NO_QUEUE)) return LH_ERR_INVALID_ARG;
  const int old = g_schedule.exchange(flags);
  if (previous) *previous = old;
  return LH_OK;
}

extern "C" int lh_attn_queue_slot(void* stream, void** slot) {
  if (!slot) return LH_ERR_INVALID_ARG;
  *slot = wq_counters(reinterpret_cast<hipStream_t>(stream));
  return *slot ? LH_OK : LH_ERR_UNSUPPORTED;
}

extern "C" int lh_dilated_scores(const void* xq, const void* xk, const void* xv, float* scores_qk, float* scores_kq,
                                 int B, int S, int H, int D, int dilation, int S_tot, float scale, int dtype,
                                 void* stream) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!valid_dtype(dtype)) return LH_ERR_INVALID_ARG;
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
                       scale > 0.f ? scale : (float)(1.0 / 11.313708498984761));
    if (rc) return rc;
    a.scores = pass == 0 ? scores_qk : scores_kq;
    a.Ho = H; a.dil = dilation; a.S_tot = S_tot;
    QPlan p;
    WorkQ wq;
    const int grid = query_grid(a.BH, a.n, st, p, wq);
    LH_DISPATCH_DTYPE(dtype, hipLaunchKernelGGL((attn_fwd_kernel<T, 1>), dim3(grid), dim3(64 * QW), 0, st, a, p, wq));
    LH_CHECK_LAUNCH();
  }
  return LH_OK;
}

namespace {
// Segments of the GLA walk.  Automatic: one per GLA_CHUNKS_PER_SEGMENT chunks
// of 64 tokens (at least one), from the sequence length alone, so that a
// sequence's walk, and with it the last bits of its bf16 scores, never depends
// on how many sequences share the launch (B, dilation, H) or on the device.
// At the reference's GLA flavor (32768 tokens, dilation 4: 128 chunks) that is
// 4 segments, 256 workgroups for 8 heads (one per CU: the scoring kernel holds
// 139 KB of LDS).  segments > 0 asks for that many (clamped to the chunk
// count).  Every segment is non-empty.
constexpr int GLA_CHUNKS_PER_SEGMENT = 32;
void gla_segments(int B, int S, int H, int dilation, int segments, int* P, int* cps) {
  (void)B;
  (void)H;
  const int T = S / dilation;
  const int nch = (T + 63) / 64;
  long long want = segments;
  if (want <= 0) want = std::max(1, nch / GLA_CHUNKS_PER_SEGMENT);
  want = std::max<long long>(1, std::min<long long>(want, nch));
  *cps = (int)((nch + want - 1) / want);
  *P = (nch + *cps - 1) / *cps;
}

int gla_check(const void* xq, const void* xk, const void* xv, const float* gk, int B, int S, int H, int D,
              int dilation, float scale) {
  if (D != LH_D) return LH_ERR_UNSUPPORTED;
  if (!xq || !xk || !xv || !gk || B <= 0 || H <= 0 || dilation <= 0 || S <= 0 || S % dilation || !(scale > 0.f))
    return LH_ERR_INVALID_ARG;
  if (!al16(xq) || !al16(xk) || !al16(xv) || (reinterpret_cast<uintptr_t>(gk) & 3u)) return LH_ERR_INVALID_ARG;
  // token offsets inside one virtual head are 32-bit
  if ((long long)S * H * D > 0x7fffffffLL || (long long)B * dilation * H * 2 > 0x7fffffffLL)
    return LH_ERR_UNSUPPORTED;
  return LH_OK;
}

long long gla_ws_bytes(int B, int H, int dilation, int P) {
  if (P <= 1) return 0;
  const long long units = (long long)B * dilation * H * 2;
  return units * (P - 1) * ((long long)GLA_WS_SEG + 1) * (long long)sizeof(float);
}
}  // namespace

extern "C" int64_t lh_gla_workspace_bytes(int B, int S, int H, int D, int dilation, int segments) {
  if (B <= 0 || H <= 0 || dilation <= 0 || S <= 0 || S % dilation || D != LH_D) return -1;
  int P, cps;
  gla_segments(B, S, H, dilation, segments, &P, &cps);
  return gla_ws_bytes(B, H, dilation, P);
}

extern "C" int lh_gla_scores(const void* xq, const void* xk, const void* xv, const float* gk, float* scores_qk,
                             float* scores_kq, int B, int S, int H, int D, int dilation, int S_tot, float scale,
                             int segments, void* workspace, int64_t workspace_bytes, int dtype, void* stream) {
  int rc = gla_check(xq, xk, xv, gk, B, S, H, D, dilation, scale);
  if (rc) return rc;
  if (!valid_dtype(dtype)) return LH_ERR_INVALID_ARG;
  if (!scores_qk || !scores_kq || S_tot < S) return LH_ERR_INVALID_ARG;
  GlaArgs a{};
  a.q = (const bf16_t*)xq; a.k = (const bf16_t*)xk; a.v = (const bf16_t*)xv; a.g = gk;
  a.sqk = scores_qk; a.skq = scores_kq;
  a.B = B; a.S = S; a.H = H; a.dil = dilation; a.T = S / dilation; a.S_tot = S_tot; a.scale = scale;
  gla_segments(B, S, H, dilation, segments, &a.P, &a.cps);
  const long long units = (long long)B * dilation * H * 2;
  if (units * a.P > 0x7fffffffLL) return LH_ERR_UNSUPPORTED;
  if (a.P > 1) {
    if (!workspace || !al16(workspace) || workspace_bytes < gla_ws_bytes(B, H, dilation, a.P))
      return LH_ERR_INVALID_ARG;
    a.ws = (float*)workspace;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  LH_DISPATCH_DTYPE(dtype, {
    if (a.P > 1) hipLaunchKernelGGL(gla_state_kernel<T>, dim3((unsigned)(units * (a.P - 1))), dim3(512), 0, st, a);
    hipLaunchKernelGGL(gla_scores_kernel<T>, dim3((unsigned)(units * a.P)), dim3(512), 0, st, a);
  });
  LH_CHECK_LAUNCH();
  return LH_OK;
}

/*
 * lighthouse_hip.h - C ABI of the gfx950 Lighthouse selection-attention library
 * (liblighthouse_hip.so).
 *
 * Every entry point:
 *   - takes plain device pointers, sizes and element strides (no framework types);
 *   - launches asynchronously on `stream` (a hipStream_t passed as void*; NULL =
 *     the default stream) and never synchronizes the host;
 *   - allocates no memory: every buffer is owned by the caller;
 *   - returns LH_OK (0) or an LH_ERR_* code (lh_strerror() names it); argument
 *     errors are detected on the host before any launch.
 *
 * Layouts (B batch, S base length, H heads, D = 128 head dim, p pooling
 * factor, L levels, S_tot = sum_l S/p^(l-1), Sp = S_tot - S, n = selected
 * length):
 *   base rows     bf16 [B, S, H, D]   (the model's xq/xk/xv, post-RoPE)
 *   pooled rows   bf16 [B, Sp, H, D]  (levels 2..L, base-first order)
 *   scores        fp32 [B, H, S_tot]  (bf16-rounded norms, widened)
 *   indices       int32 [B, H, n]     pyramid indices in causal order
 *   inverse       int32 [B, H, S_tot] position in the selected sequence or -1
 *   selected rows bf16 [B, H, n, D];  lse / delta fp32 [B, H, n]
 *   layer output  bf16 [B, H, S, D]
 *
 * Citations are to the reference repository (ighoshsubho/lighthouse-attention).
 */
#ifndef LIGHTHOUSE_HIP_H
#define LIGHTHOUSE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LH_OK 0
#define LH_ERR_INVALID_ARG 1  /* bad size, null pointer or unsupported shape */
#define LH_ERR_DOMAIN 2       /* geometry the reference asserts on or overruns (strict mode) */
#define LH_ERR_LAUNCH 3       /* the HIP runtime refused a launch */
#define LH_ERR_UNSUPPORTED 4  /* shape beyond this build's limits (e.g. D != 128) */
#define LH_ERR_RUNTIME 5      /* a HIP runtime call (synchronize, copy, symbol lookup) failed */

/* The ABI this header declares; lh_abi_version() of a matching library returns it. */
#define LH_ABI_VERSION 9

#define LH_DTYPE_BF16 0       /* row element type: bfloat16 (the reference configs) */
#define LH_DTYPE_F16 1        /* row element type: IEEE half */

#define LH_TIE_REFERENCE 0    /* the reference network: strict compare-exchange only */
#define LH_TIE_LOWER_INDEX 1  /* ties ordered by lower level-local index */

/* Human-readable name of a return code. */
const char *lh_strerror(int rc);

/* ABI version of the library (LH_ABI_VERSION of the header it was built
 * with; bumped on any signature or error-code change). */
int lh_abi_version(void);

/*
 * Tiling of the selection and the selected length.
 * Replaces compute_output_indices_selection (src/lighthouse_selection_cuda.py:346-357)
 * and the tiling/asserts of LighthouseSelectionQkKqChunkedTopkNvrtc.forward
 * (src/lighthouse_selection_cuda.py:370-397).
 * strict = 1 reproduces the reference's domain (LH_ERR_DOMAIN outside it);
 * strict = 0 admits any shape with per-tile compaction.
 * Any output pointer may be NULL.
 */
int lh_select_geometry(int S, int L, int p, int topk, int strict,
                       int *num_tiles, int *nodes_per_tile, int *per_tile, int *S_sel);

/*
 * Norm scorer + Q/K/V pyramid, one streaming pass.
 * Replaces DialatedLighthouseNormScorer.forward (src/lighthouse_selection.py:589-616)
 * and the pyramid half of DilatedLighthouseScorer.forward (:655-689).
 *   xq, xk, xv      base rows of element type dtype (LH_DTYPE_BF16 / _F16),
 *                   strides (sb, ss, sh) in elements, D contiguous
 *   pq, pk, pv      pooled rows (dtype) written for levels 2..L, strides (pb, ps, ph)
 *   scores_qk/_kq   fp32 [B, H, S_tot] contiguous
 *   base_scores_given = 0: base-level scores are the L2 norms of xq (qk) and
 *     xk (kq) rounded to dtype (torch's norm of such rows); = 1: base-level
 *     scores are already in scores_* (written by lh_dilated_scores or
 *     lh_gla_scores) and only the max-pooled levels are made.
 * Every row-reading entry point of this library below takes the same dtype
 * argument (its rows, outputs and rounding follow it; sums are fp32);
 * the rotary entry points are bf16 only.
 */
int lh_pyramid_fwd(const void *xq, const void *xk, const void *xv,
                   int64_t sb, int64_t ss, int64_t sh,
                   void *pq, void *pk, void *pv,
                   int64_t pb, int64_t ps, int64_t ph,
                   float *scores_qk, float *scores_kq,
                   int B, int S, int H, int D, int L, int p,
                   int base_scores_given, int dtype, void *stream);

/*
 * Rotary embedding fused into the norm-scorer pyramid pass.
 * Replaces torchtitan's apply_rotary_emb on q and k (the caller of
 * selection_attn, lighthouse-attention.patch:707-712) followed by
 * DialatedLighthouseNormScorer.forward (src/lighthouse_selection.py:589-616):
 * the rows are read once, unrotated.
 *   xq, xk, xv      bf16 rows of the q/k/v projections (q, k unrotated), strides
 *                   (sb, ss, sh), D contiguous; e.g. column blocks of the fused
 *                   [q | k | v] projection output
 *   freqs           fp32 [>= S, D/2, 2] (cos, sin) per position and pair
 *   rq, rk          bf16 rotated q, k base rows written here, strides (rb, rs, rh);
 *                   every row is rounded to bf16 once, and the scores and pooled
 *                   rows are those of the rounded rows (the same bits as rotating
 *                   first and then calling lh_pyramid_fwd)
 *   the rest as lh_pyramid_fwd with base_scores_given = 0
 */
int lh_rope_pyramid_fwd(const void *xq, const void *xk, const void *xv,
                        int64_t sb, int64_t ss, int64_t sh,
                        const float *freqs,
                        void *rq, void *rk, int64_t rb, int64_t rs, int64_t rh,
                        void *pq, void *pk, void *pv,
                        int64_t pb, int64_t ps, int64_t ph,
                        float *scores_qk, float *scores_kq,
                        int B, int S, int H, int D, int L, int p, void *stream);

/*
 * Dilated scorer base scores: ||causal_attn(q,k,v)||_2 and ||causal_attn(k,q,v)||_2
 * over the dilated virtual heads, written to scores_qk/_kq[:, :, 0:S].
 * Replaces the two SDPA calls and norms of DilatedLighthouseScorer.forward
 * (src/lighthouse_selection.py:638-653).  Inputs are contiguous [B, S, H, D].
 * scale: the softmax scale (<= 0: 1/sqrt(D)); a head dim padded with zeros to D
 * passes 1/sqrt(its own width).
 */
int lh_dilated_scores(const void *xq, const void *xk, const void *xv,
                      float *scores_qk, float *scores_kq,
                      int B, int S, int H, int D, int dilation, int S_tot, float scale, int dtype,
                      void *stream);

/*
 * GLA scorer base scores: the L2 norms of the two simple gated linear
 * attention outputs o = chunk_simple_gla(q, k, v, g, scale) and
 * chunk_simple_gla(k, q, v, g, scale) over the dilated virtual heads (each
 * output rounded to dtype first, the norm rounded to dtype), written to
 * scores_qk/_kq[:, :, 0:S].
 * Replaces the two fla chunk_simple_gla calls and norms of
 * DilatedLighthouseGLAScorer.forward (src/lighthouse_selection.py:713-734).
 *   xq, xk, xv  dtype [B, S, H, D] contiguous; gk fp32 [B, S, H] contiguous log gates
 *               (the running state is fp32; its copy used as the inter-chunk MFMA
 *               operand is rounded to dtype, so with fp16 a state entry beyond
 *               fp16's range, 65504, becomes infinite there)
 *   (token t of head h is position t / dilation of virtual head (t % dilation) * H + h)
 *   segments   <= 0: automatic, one per 32 chunks of 64 tokens (at least one),
 *              from the per-sequence length S / dilation alone, so a sequence's
 *              scores do not depend on the batch or head count around it; else
 *              the number of sequence segments walked in parallel (clamped to
 *              the 64-token chunk count).  Segment s starts
 *              from the combined final states of segments 0..s-1, which a first
 *              pass computes; results agree with the one-segment walk to fp32
 *              rounding of the state (the rounded scores may differ in the last bit).
 *   workspace  device buffer of lh_gla_workspace_bytes(...) bytes (16-byte aligned),
 *              may be NULL when that size is 0; workspace_bytes is its size.
 * Then lh_pyramid_fwd with base_scores_given = 1 pools the levels.
 */
int lh_gla_scores(const void *xq, const void *xk, const void *xv, const float *gk,
                  float *scores_qk, float *scores_kq,
                  int B, int S, int H, int D, int dilation, int S_tot, float scale,
                  int segments, void *workspace, int64_t workspace_bytes, int dtype, void *stream);

/*
 * Workspace bytes lh_gla_scores needs for this geometry and `segments` (0 when
 * it walks one segment; -1 for an invalid geometry).  Host-only, no GPU call.
 */
int64_t lh_gla_workspace_bytes(int B, int S, int H, int D, int dilation, int segments);

/*
 * Hierarchical per-tile top-k selection, emitted in causal order.
 * Replaces lighthouse_selection_chunked_topk_kernel + torch.sort/gather
 * (src/lighthouse_selection_cuda.py:114-331, :399-427).
 *   scores_qk/_kq  fp32 [B, H, S_tot] contiguous
 *   indices        int32 [B, H, S_sel] (S_sel from lh_select_geometry)
 *   inverse        int32 [B, H, S_tot] or NULL
 *   tie_mode       LH_TIE_REFERENCE or LH_TIE_LOWER_INDEX
 */
int lh_select_topk(const float *scores_qk, const float *scores_kq,
                   int32_t *indices, int32_t *inverse,
                   int B, int H, int S, int L, int p, int topk,
                   int tie_mode, int strict, void *stream);

/*
 * inverse[b,h,r] = s where indices[b,h,s] == r, else -1.  (Device helper for
 * callers holding only `indices`, e.g. scatter_to_base_sequence.)
 * Entries outside [0, S_tot) are skipped.  Indices must be unique per (b, h):
 * for a row named twice, one of its positions (unspecified which) is kept, so
 * the fan-out and its adjoint would count that row once.  lh_check_indices
 * detects duplicates.
 */
int lh_build_inverse(const int32_t *indices, int n, int32_t *inverse, int S_tot,
                     int B, int H, void *stream);

/*
 * Validation of an index array, for callers' debug/check modes (no counterpart
 * in the reference, whose Python asserts shapes only).
 *   indices  int32 [B, H, n] contiguous
 *   counts   device int32[2], written: counts[0] = entries outside [lo, hi),
 *            counts[1] = duplicate entries within a (b, h) (0 unless marks given;
 *            with lo = -1, entries equal to -1 are empty slots, never duplicates)
 *   marks    device int32 [B, H, hi - lo] workspace for the duplicate count, or NULL
 * Asynchronous like every entry point: read `counts` after the stream has run.
 */
int lh_check_indices(const int32_t *indices, int B, int H, int n, int lo, int hi,
                     int32_t *marks, int32_t *counts, void *stream);

/*
 * Causal attention over gathered rows, forward.
 * Replaces the three torch.gather calls + self.attention(...)
 * (src/lighthouse_selection.py:800-815).
 * Row r of (b, h) is read from
 *   base + b*sb + r*ss + h*sh            if r <  split
 *   pool + b*pb + (r-split)*ps + h*ph    if r >= split
 * where r = indices[b,h,s] (or r = s when indices == NULL).
 * Precondition (not checked on the device): 0 <= indices[b,h,s] < split + P,
 * P the number of pooled rows behind `pool` (S_tot - S for a pyramid); the
 * kernels read row r unguarded.  lh_check_indices validates an index array.
 *   out  bf16 [B, H, n, D];  lse fp32 [B, H, n] (log2-domain: m*log2(e)+log2(sum),
 *        sum = the row sum of the bf16-rounded probabilities that weight V, so
 *        the weights of each output row sum to 1 up to fp32 accumulation)
 * With more blocks than CUs this launch and the backward's run one workgroup
 * per CU, taking blocks from a host-packed plan or from work-queue counters
 * that live in the library's device memory, one slot per (device, stream),
 * which each launch leaves cleared.  Launches on different streams therefore
 * never share counters.  A launch made while its stream is being captured into
 * a graph gets a slot of its own, used by no other launch, so captured graphs
 * may be replayed on any stream, beside eager launches and other graphs; only
 * a graph replayed beside itself (two replays of it in flight at once) races.
 * Each persistent launch checks that its blocks added up and otherwise flags
 * its slot (a slot not cleared at launch: a launch that never finished, or a
 * replay that overlapped itself); lh_attn_status reports and resets it.
 */
int lh_attn_fwd(const void *q, const void *k, const void *v, int64_t sb, int64_t ss, int64_t sh,
                const void *qp, const void *kp, const void *vp, int64_t pb, int64_t ps, int64_t ph,
                int split, const int32_t *indices, int B, int H, int n, int D, float scale,
                void *out, float *lse, int dtype, void *stream);

/*
 * Causal attention backward over gathered rows (deterministic: dK/dV per key
 * block, dQ per query block, each output element written by one workgroup;
 * block scheduling as lh_attn_fwd).  Replaces the SDPA backward and the
 * gather backward's row selection (src/lighthouse_selection.py:800-815).
 *   dout   bf16 [B, H, n, D] (from lh_scatter_bwd); lse, delta fp32 [B, H, n]
 *   dq, dk, dv bf16 [B, H, n, D] in selected order
 * With indices, n must be >= 8 (LH_ERR_UNSUPPORTED otherwise); every selected
 * length of a Lighthouse pyramid is.  Index precondition as lh_attn_fwd.
 */
int lh_attn_bwd(const void *q, const void *k, const void *v, int64_t sb, int64_t ss, int64_t sh,
                const void *qp, const void *kp, const void *vp, int64_t pb, int64_t ps, int64_t ph,
                int split, const int32_t *indices, int B, int H, int n, int D, float scale,
                const void *dout, const float *lse, const float *delta,
                void *dq, void *dk, void *dv, int dtype, void *stream);

/*
 * The two independent halves of lh_attn_bwd (same arguments), for callers that
 * schedule them separately, e.g. on two streams: the key-stationary dK/dV
 * kernel and the query-stationary dQ kernel.
 */
int lh_attn_bwd_dkdv(const void *q, const void *k, const void *v, int64_t sb, int64_t ss, int64_t sh,
                     const void *qp, const void *kp, const void *vp, int64_t pb, int64_t ps, int64_t ph,
                     int split, const int32_t *indices, int B, int H, int n, int D, float scale,
                     const void *dout, const float *lse, const float *delta,
                     void *dk, void *dv, int dtype, void *stream);
int lh_attn_bwd_dq(const void *q, const void *k, const void *v, int64_t sb, int64_t ss, int64_t sh,
                   const void *qp, const void *kp, const void *vp, int64_t pb, int64_t ps, int64_t ph,
                   int split, const int32_t *indices, int B, int H, int n, int D, float scale,
                   const void *dout, const float *lse, const float *delta,
                   void *dq, int dtype, void *stream);

/*
 * Work-queue faults of the persistent attention launches (lh_attn_fwd,
 * lh_attn_bwd*, lh_dilated_scores) on the current device since the last call.
 * Waits for the device to go idle (hipDeviceSynchronize), then counts the
 * counter slots that a launch flagged (its blocks did not add up: entries were
 * skipped because the slot was not clear at launch) or that are not clear now
 * (with no launch in flight every slot must be zero), and resets them, so the
 * next launch on them is whole.  *faults = 0: no fault.  Call it outside graph
 * capture and with no launch of this library being issued from another host
 * thread.  The reference has no such state (its SDPA has no persistent
 * launches); this is the check behind the Python layer's check mode
 * (LH_CHECK_INDICES=1).
 */
int lh_attn_status(int *faults);

/*
 * Diagnostics: the device address of the counter slot (32 unsigned words) that
 * persistent launches on `stream` use on the current device, assigned on first
 * use; LH_ERR_UNSUPPORTED when every slot is taken.  Tests use it to plant a
 * dirty slot.  No counterpart in the reference.
 */
int lh_attn_queue_slot(void *stream, void **slot);

/*
 * Scheduling of the attention launches (lh_attn_fwd, lh_attn_bwd*,
 * lh_dilated_scores) in this process, for A/B measurement: 0 (the default)
 * lets each launch choose a packed query-block plan, per-XCD work queues or one
 * block per workgroup by its shape; LH_SCHED_NO_PLAN never uses a plan,
 * LH_SCHED_NO_QUEUE never uses the queues; both together give one block per
 * workgroup everywhere.  Outputs are bit-identical under every setting (each
 * block's arithmetic is the same).  *previous (if not NULL) receives the old
 * flags; unknown bits give LH_ERR_INVALID_ARG.  Takes effect for launches issued
 * after the call; a graph keeps the schedule it was captured with.  No
 * counterpart in the reference.
 */
#define LH_SCHED_NO_PLAN 1
#define LH_SCHED_NO_QUEUE 2
int lh_attn_set_schedule(int flags, int *previous);

/*
 * Fan-out of each selected row onto the base positions it stands for:
 * out[b,h,t] = sum over levels l of attn[b,h,inverse[b,h,off_l + (t+1)/c_l - 1]].
 * Replaces _scatter_fanout_fwd_kernel / _ScatterToBaseAutograd.forward
 * (src/lighthouse_selection.py:408-459, :519-550) without atomics.
 *   attn bf16 [B, H, n, D]; out bf16 [B, H, S_out, D] logically.  When S_out > S, a row
 *   t >= S receives the coarse-level entries whose span [(i+1)c_l - 1, (i+2)c_l - 2]
 *   reaches t (as in the reference); rows no span reaches are zero.  `inverse` entries
 *   must be -1 or < n.  Layout:
 *   element (b, h, t, :) at out + b*ob + h*oh + t*os (D contiguous): (H*S_out*D, S_out*D, D)
 *   for [B, H, S_out, D] storage, (S_out*H*D, D, H*D) for [B, S_out, H, D] storage.
 */
int lh_scatter_fwd(const void *attn, const int32_t *inverse, void *out, int64_t ob, int64_t oh, int64_t os,
                   int B, int H, int S, int S_out, int n, int D, int L, int p, int dtype, void *stream);

/*
 * Adjoint of the fan-out: dattn[s] = sum of dout over the span of entry s,
 * plus delta[s] = sum_d bf16(dattn[s,d]) * o[s,d] for the attention backward
 * (delta is skipped when o or delta is NULL).
 * Replaces _scatter_fanout_bwd_kernel (src/lighthouse_selection.py:462-514, :552-576).
 *   dout bf16 [B, H, S_out, D] logically, element (b, h, t, :) at dout + b*db + h*dh + t*ds
 */
int lh_scatter_bwd(const void *dout, int64_t db, int64_t dh, int64_t ds, const int32_t *indices, const void *o,
                   void *dattn, float *delta,
                   int B, int H, int S, int S_out, int n, int D, int L, int p, int dtype, void *stream);

/*
 * Pyramid backward: dX[b,t,h] = g[inverse(t)] + sum_{l>=2} g[inverse(off_l + t/c_l)] / c_l
 * for X in {q, k, v} at once (any of the three may be NULL).
 * Replaces the autograd of torch.gather + torch.cat + mean
 * (src/lighthouse_selection.py:604-614, :800-813).
 *   gq, gk, gv  bf16 selected-space grads, strides (gb, gh, gs) in elements
 *   inverse     int32 [B, H, S_tot]; NULL means the identity (g indexed by pyramid row)
 *   dxq/dxk/dxv bf16 [B, S, H, D] contiguous
 */
int lh_pyramid_bwd(const void *gq, const void *gk, const void *gv,
                   int64_t gb, int64_t gh, int64_t gs,
                   const int32_t *inverse,
                   void *dxq, void *dxk, void *dxv,
                   int B, int S, int H, int D, int L, int p, int dtype, void *stream);

/*
 * Pyramid backward with the rotary embedding's backward fused in: as
 * lh_pyramid_bwd, then dxq and dxk are rotated by -theta (the adjoint of the
 * forward rotation; torchtitan apply_rotary_emb's autograd) in fp32 before the
 * one rounding.  Outputs have strides (ob, os, oh) in elements, D contiguous;
 * e.g. the column blocks of the [q | k | v] projection-output gradient.
 *   freqs   fp32 [>= S, D/2, 2], as in lh_rope_pyramid_fwd
 */
int lh_pyramid_rope_bwd(const void *gq, const void *gk, const void *gv,
                        int64_t gb, int64_t gh, int64_t gs,
                        const int32_t *inverse, const float *freqs,
                        void *dxq, void *dxk, void *dxv, int64_t ob, int64_t os, int64_t oh,
                        int B, int S, int H, int D, int L, int p, void *stream);

/*
 * Transformer-block kernels of the Llama3 model that hosts the layer
 * (lighthouse-attention.patch:583-769 over torchtitan's llama3 model, which
 * is upstream and not vendored).  They replace torch op chains, not reference
 * kernels; each names the chain it replaces.
 */

/*
 * Rotary embedding fused with the q/k/v split of the projection output.
 * Replaces apply_rotary_emb (torchtitan llama3 model: view_as_complex * freqs_cis,
 * fp32, cast back) on wq(x), wk(x) plus the split of wv(x) (patch :707-724).
 *   x        bf16 rows [B*S] of (Hq + 2 Hkv) * D elements, row stride xs, laid out
 *            [q heads | k heads | v heads]
 *   freqs    fp32 [>= S, D/2, 2] (cos, sin) of position t and pair j
 *   q, k, v  bf16 [B, S, Hq|Hkv, D] contiguous; q and k rotated, v copied
 */
int lh_rope_qkv_fwd(const void *x, int64_t xs, const float *freqs, void *q, void *k, void *v,
                    int B, int S, int Hq, int Hkv, int D, void *stream);

/*
 * Adjoint: dx = [R(-angle) dq | R(-angle) dk | dv] in the projection-output layout.
 *   strides  9 int64: (batch, seq, head) element strides of dq, dk, dv (D contiguous)
 */
int lh_rope_qkv_bwd(const void *dq, const void *dk, const void *dv, const int64_t *strides,
                    const float *freqs, void *dx, int64_t xs, int B, int S, int Hq, int Hkv, int D,
                    void *stream);

/*
 * RMSNorm over rows of dim elements (dim a multiple of 8, <= 4096):
 * y = bf16((x * r) * w), r = 1/sqrt(mean(x^2) + eps), rstd[row] = r.
 * Replaces nn.RMSNorm (torch.rms_norm) of the block's attention_norm, ffn_norm and norm.
 */
int lh_rmsnorm_fwd(const void *x, const void *w, void *y, float *rstd, int64_t rows, int dim, float eps,
                   void *stream);

/*
 * Residual add fused with the RMSNorm that follows it: h = bf16(x + r) is written
 * out, and y = RMSNorm(h) as lh_rmsnorm_fwd.  Replaces `h = x + attn(...)` followed
 * by `ffn_norm(h)` (and the next block's `attention_norm`) in the Llama3 block.
 */
int lh_add_rmsnorm_fwd(const void *x, const void *r, const void *w, void *h, void *y, float *rstd,
                       int64_t rows, int dim, float eps, void *stream);

/*
 * RMSNorm backward: dx = r g - x r^3 mean(g x) (+ dres) with g = dy w; dw = sum_rows dy x r.
 * dres (optional, bf16 like dx) is the gradient reaching x through a residual branch,
 * added in fp32 before the rounding.  dw_part is caller workspace, fp32 [dim, parts];
 * dw is bf16 [dim].
 */
int lh_rmsnorm_bwd(const void *dy, const void *x, const void *w, const float *rstd, const void *dres,
                   void *dx, void *dw, float *dw_part, int parts, int64_t rows, int dim, void *stream);

/*
 * lh_rmsnorm_bwd without the dw_part workspace: the per-block dw partials live in
 * a static device array of the library (256 partials x 4096 columns fp32 = 4 MiB per
 * GPU, held until the process ends), so this entry point allocates nothing and
 * takes no workspace.  No counterpart in the reference; it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same results as lh_rmsnorm_bwd with parts = 256.
 * dim <= 4096 (LH_ERR_UNSUPPORTED otherwise).  All calls on one GPU share the
 * array: calls that overlap on one GPU (other streams, other threads) race.
 */
int lh_rmsnorm_bwd_noalloc(const void *dy, const void *x, const void *w, const float *rstd, const void *dres,
                           void *dx, void *dw, int64_t rows, int dim, void *stream);

/*
 * SwiGLU on the fused [h1 | h3] projection (rows of 2F): a = bf16(bf16(silu(h1)) h3).
 * Replaces F.silu(w1(x)) * w3(x) of FeedForward (torchtitan llama3 model).
 */
int lh_swiglu_fwd(const void *h, void *a, int64_t rows, int F, void *stream);

/* SwiGLU backward into the fused layout: dh = [dh1 | dh3] (rows of 2F). */
int lh_swiglu_bwd(const void *da, const void *h, void *dh, int64_t rows, int F, void *stream);

/*
 * Sum of split-K partial products: out[i] = bf16(sum_s part[s][i]) for the
 * projections' weight gradients computed in token slices (fp32 [splits, n],
 * n a multiple of 8).  Replaces part.sum(0).to(bfloat16).
 */
int lh_splitk_sum(const float *part, void *out, int splits, int64_t n, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LIGHTHOUSE_HIP_H */

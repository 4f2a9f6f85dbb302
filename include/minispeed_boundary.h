/*
 * minispeed_boundary.h — C ABI of the MI355X (gfx950) gradient-accumulation
 * boundary step: the flatten / inf-nan / unscale / global-norm / clip /
 * AdamW / master->model cast sequence that minispeed runs in
 * DeepSpeedEngine._take_optimizer_step (minispeed/engine.py:268-322).
 *
 * Conventions
 *   - Every pointer argument is caller-owned memory. Device pointers are
 *     marked [dev]; everything else is host memory read during the call.
 *   - Every entry point is asynchronous on the `stream` argument (a
 *     hipStream_t passed as void*; NULL is the legacy default stream) and
 *     allocates nothing.
 *   - Return value: 0 on success, a negative MS_E* code for an argument
 *     error detected on the host (nothing was launched), or a positive
 *     hipError_t from the launch.  ms_error_string() names both kinds.
 *   - Flat indices are "group coordinates": element k of a parameter that
 *     starts at flat offset o has index o + k (minispeed/flat.py:81-86).
 *     Arrays passed as `float* x` together with a range [begin, end) hold
 *     index i at x[i - begin].
 *   - Thread-compatible, not thread-safe: concurrent calls on different
 *     streams must use different output buffers.
 */
#ifndef MINISPEED_BOUNDARY_H
#define MINISPEED_BOUNDARY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MS_ABI_VERSION 8

/* groups one ms_boundary_scalars_noalloc call can scan, and the tiles
 * (MS_SCAN_TILE flat indices each) of the largest one: its static scratch
 * holds MS_SCRATCH_MAX_GROUPS x ms_stats_blocks() partial slots and
 * MS_SCRATCH_MAX_TILES tile slots of 12 bytes each (25.5 MiB) */
#define MS_SCRATCH_MAX_GROUPS 8
#define MS_SCRATCH_MAX_TILES (1 << 21)

/* flat indices per K1 tile (one wave of 64 lanes scans one tile) */
#define MS_SCAN_TILE 2048

/* element types of ragged gradient / model storage */
enum {
  MS_DTYPE_F32 = 0,
  MS_DTYPE_F16 = 1,
  MS_DTYPE_BF16 = 2
};

/* what ms_grad_stats does to each widened gradient with `grad_scale`
 * (ms_fused_adamw accepts NONE and DIVIDE) */
enum {
  MS_SCALE_NONE = 0,      /* g                                           */
  MS_SCALE_DIVIDE = 1,    /* g / grad_scale, IEEE (unscale_grads,
                             flat.py:243-247); grad_scale > 0            */
  MS_SCALE_MULTIPLY = 2   /* g * grad_scale, one rounding (scale_grads,
                             flat.py:249-257)                            */
};

/* host-side argument errors (nothing launched) */
enum {
  MS_OK = 0,
  MS_EINVAL = -1,   /* bad size, range, dtype or NULL where required */
  MS_ETABLE = -2,   /* segment count out of range */
  MS_EBLOCKS = -3,  /* partial-sum workspace smaller than ms_stats_blocks(),
                       or tile workspace smaller than the scanned range's tiles */
  MS_ESCRATCH = -4  /* more groups than MS_SCRATCH_MAX_GROUPS, or a group of
                       more than MS_SCRATCH_MAX_TILES tiles */
};

/*
 * One contiguous piece of a flat group: flat indices [begin, begin+numel).
 * `grad`  : storage of those elements' gradients in the group's grad dtype
 *           (param.grad viewed flat, advanced to `begin`), or NULL when the
 *           parameter has no gradient (it contributes zeros, flat.py:209-211)
 *           or for the padding tail.
 * `model` : storage of the model-dtype parameter elements to overwrite with
 *           the cast of the updated fp32 master (flat.py:148-154), or NULL
 *           when nothing is written (padding; ZeRO-3 while not gathered).
 * A table passed to a kernel lives in device memory, is sorted by `begin`,
 * and tiles the kernel's range exactly (no gaps, no overlap).  `begin` and
 * the two pointers may have any element alignment (a tensor of odd size
 * shifts every later segment of a packed flat layout): results do not
 * depend on it; speed does somewhat (16-byte aligned storage starting on
 * the flat space's 16-byte grid is the fastest case).
 * Replaces the per-parameter (offset, numel, param) list walked by
 * FlatParamGroup.flatten_grads / copy_flat_to_model (flat.py:78-86, 196-213,
 * 133-154).
 */
typedef struct ms_segment {
  int64_t begin;
  int64_t numel;
  const void* grad;
  void* model;
} ms_segment_t;

/*
 * Result of the boundary reduction (K2), written to device memory and read
 * back by the host with one copy per boundary.
 */
typedef struct ms_step_scalars {
  uint32_t overflow;      /* any inf/nan in the scanned grads, pre-unscale
                             (precision.py:79-87, engine.py:275)            */
  uint32_t clip_applied;  /* norm > max_norm and coef != 1
                             (stage_1_and_2.py:123-126, flat.py:252-253)     */
  float sumsq;            /* fp32 sum over groups of per-group sum of
                             squares of the unscaled owned grads
                             (stage_1_and_2.py:114-116)                     */
  float norm;             /* sqrtf(sumsq) (stage_1_and_2.py:121)            */
  float coef;             /* fp32(max_norm / (norm + 1e-6)) if clip_applied,
                             else 1 (stage_1_and_2.py:124)                  */
  uint32_t ready;         /* 0 in K2's device output; in its host copy set
                             to 1 after every other field is visible to the
                             host (see ms_norm_clip)                        */
  double coef64;          /* the same coefficient before fp32 rounding      */
  double next_scale;      /* loss scale after DynamicLossScaler.update
                             (precision.py:50-62)                           */
  int64_t next_good_steps;
  int64_t next_skipped_steps;
} ms_step_scalars_t;

/*
 * AdamW hyper-parameters for one group and one step, already rounded the
 * way minispeed's torch op sequence rounds them (optim/adam.py:80-91):
 * every scalar is the fp32 rounding of the double the reference computes.
 */
typedef struct ms_adamw_params {
  float neg_lr;          /* fp32(-lr)                  addcdiv value      */
  float decay_alpha;     /* fp32(-lr * weight_decay)   add_ alpha         */
  float beta1;           /* fp32(beta1)                mul_               */
  float one_minus_beta1; /* fp32(1 - beta1)            add_ alpha         */
  float beta2;           /* fp32(beta2)                mul_               */
  float one_minus_beta2; /* fp32(1 - beta2)            addcmul value      */
  float bias_c1;         /* fp32(1 - beta1**step)      m / bias_c1        */
  float bias_c2;         /* fp32(1 - beta2**step)      v / bias_c2        */
  float eps;             /* fp32(eps)                  add_               */
  float grad_scale;      /* loss scale to divide ragged grads by          */
  int32_t decay;         /* weight_decay != 0 (adam.py:81)                */
  int32_t unscale;       /* MS_SCALE_DIVIDE: divide ragged grads by
                            grad_scale (flat.py:247); or MS_SCALE_NONE   */
} ms_adamw_params_t;

/* MS_ABI_VERSION of the loaded library. */
int ms_abi_version(void);

/* Static text for a return code of this library. */
const char* ms_error_string(int code);

/* Number of per-group partial slots K2 reduces (a constant, 16384).  K1
 * writes one statistics slot per tile of MS_SCAN_TILE flat indices and folds
 * the tiles into these slots in a fixed order (as ms_reduce_tile_stats), so
 * the norm's reduction order is a pure function of the layout and the norm
 * is run-to-run deterministic. */
int ms_stats_blocks(void);

/*
 * K1 — ragged gradient scan.  Replaces FlatParamGroup.flatten_grads
 * (flat.py:196-213), has_overflow on the flat grad (precision.py:79-87),
 * unscale_grads (flat.py:243-247), scale_grads (flat.py:249-257) and
 * local_grad_sumsq (flat.py:232-234).
 *
 * Scans flat indices [begin, end) through `segs` [dev] (`nseg` entries,
 * grad dtype `grad_dtype`) in tiles of MS_SCAN_TILE indices, tile t covering
 * [begin + t*MS_SCAN_TILE, min(begin + (t+1)*MS_SCAN_TILE, end)):
 *   - g = the exact widening fp32(grad), then per `unscale`
 *     (MS_SCALE_*): unchanged, / grad_scale (IEEE division) or
 *     * grad_scale (one rounded multiply);
 *   - flat_grad [dev, optional]: flat_grad[i - begin] = g for every i;
 *   - statistics (block_sumsq != NULL): tile_flag[t] != 0 iff some grad
 *     element of tile t is inf/nan, tested on the raw stored value (before
 *     unscale); tile_sumsq[t] = the fp64 sum of g*g over the tile's
 *     elements inside the owned range [own_begin, own_end), added in a
 *     fixed order (64 lanes, each its own elements in index order, then a
 *     fixed tree).  tile_sumsq / tile_flag [dev] need ntiles >=
 *     ceil((end - begin) / MS_SCAN_TILE) slots (the rest are left alone).
 *     The tiles are then folded into block_sumsq / block_flag [dev]
 *     (nblk >= ms_stats_blocks() slots, all written) exactly as
 *     ms_reduce_tile_stats folds them.
 * The statistics do not depend on flat_grad: with and without it the slots
 * get the same bits.  With block_sumsq == NULL (then tile_sumsq, tile_flag
 * and block_flag must be NULL too) the call is a pure ragged flatten
 * (FlatParamGroup.copy_model_to_flat, flat.py:115-131).  flat_grad may be the
 * storage of a single F32 segment spanning [begin, end): each element is
 * read before it is written, by the same lane, so the call then scales the
 * buffer in place (unscale_grads / scale_grads).
 */
int ms_grad_stats(const ms_segment_t* segs, int32_t nseg, int32_t grad_dtype,
                  int64_t begin, int64_t end, int64_t own_begin,
                  int64_t own_end, int32_t unscale, float grad_scale,
                  float* flat_grad, double* tile_sumsq, uint32_t* tile_flag,
                  int64_t ntiles, double* block_sumsq, uint32_t* block_flag,
                  int32_t nblk, void* stream);

/*
 * K2 — global norm, clip coefficient, skip and loss-scale decision.
 * Replaces global_overflow (precision.py:90-92), ZeROOptimizer.clip_gradients
 * (stage_1_and_2.py:105-128) and DynamicLossScaler.update
 * (precision.py:50-62).  One block; fixed reduction order.
 *
 * block_sumsq / block_flag [dev]: ngroups x nblk partials from K1 (group g
 * at offset g*nblk).  Per group the fp64 partials are summed and rounded to
 * fp32; the group sums are added in group order in fp32.  Clipping applies
 * when has_clip and norm > max_norm (double compare), with
 * coef64 = max_norm / (norm + 1e-6) and clip_applied = (coef64 != 1).
 * The scaler fields are the state before this boundary.
 * out [dev] receives an ms_step_scalars_t.
 * out_host [pinned host memory, optional] receives the same struct with
 * `ready` = 1, written after every other field is visible to the host: a
 * caller that set out_host->ready to 0 before this call can poll that word
 * and read the struct once it is 1, while later work on the stream keeps
 * running, with no copy and no event in the stream (the one read-back of
 * engine.py:278-322's two syncs).  Waiting for the kernel's completion
 * (an event, a stream synchronisation) also gives the whole struct.
 */
int ms_norm_clip(const double* block_sumsq, const uint32_t* block_flag,
                 int32_t nblk, int32_t ngroups, int32_t has_clip,
                 double max_norm, int32_t scaler_enabled, double scale,
                 int64_t good_steps, int64_t skipped_steps, int64_t window,
                 double min_scale, double max_scale, ms_step_scalars_t* out,
                 ms_step_scalars_t* out_host, void* stream);

/*
 * K3 — fused AdamW over the owned range [begin, end) plus the cast of the
 * updated masters into the model parameters.  Replaces FlatAdam.step
 * (optim/adam.py:59-93), the clip multiply (flat.py:249-257) and
 * copy_flat_to_model (flat.py:133-154; the ZeRO-3 placeholder refresh of
 * stage_3.py:88-110).
 *
 * master, exp_avg, exp_avg_sq [dev]: fp32, index i at [i - begin].
 * flat_grad [dev, optional]: unscaled fp32 grads at [i - begin]; when NULL
 *   the grads are read from segs[].grad (grad_dtype) and divided by
 *   hp->grad_scale when hp->unscale.
 * segs [dev]: tiles [begin, end); segs[].model (model_dtype) receives the
 *   cast of the updated master (round to nearest even).
 * scalars [dev]: K2's output.  When scalars->overflow is set the kernel
 *   returns without touching memory (the skipped step, engine.py:278-293);
 *   when scalars->clip_applied the grads are multiplied by scalars->coef.
 * hp [host]: this step's rounded hyper-parameters.
 */
int ms_fused_adamw(float* master, float* exp_avg, float* exp_avg_sq,
                   const float* flat_grad, const ms_segment_t* segs,
                   int32_t nseg, int32_t grad_dtype, int32_t model_dtype,
                   int64_t begin, int64_t end, const ms_adamw_params_t* hp,
                   const ms_step_scalars_t* scalars, void* stream);

/*
 * K4 — cast fp32 masters into model-dtype storage: flat [dev] holds index i
 * at flat[i - begin]; every segment with a non-NULL `model` inside
 * [begin, end) is written.  Replaces copy_flat_to_model (flat.py:133-154)
 * for the ZeRO-3 gather/free casts (stage_3.py:67-110) and the skip path.
 */
int ms_cast_to_model(const float* flat, int64_t begin, int64_t end,
                     const ms_segment_t* segs, int32_t nseg,
                     int32_t model_dtype, void* stream);

/*
 * K5 — opt-in contiguous gradients: dst[i] = (first ? 0 : dst[i]) +
 * (float)src[i] for i in [0, n), dst [dev] fp32, src [dev] of src_dtype.
 * Called once per parameter per micro-batch (a post-accumulate-grad hook),
 * it replaces autograd's accumulation into param.grad across the
 * micro-batches of a window (engine.py:235-251) followed by flatten_grads
 * (flat.py:196-213), accumulating in fp32 instead of the parameter dtype.
 * Not bitwise the reference by design: minispeed has no such mode.
 */
int ms_accumulate_grad(float* dst, const void* src, int32_t src_dtype, int64_t n,
                       int32_t first, void* stream);

/* One gradient of a batched K5 call: dst [dev] fp32, src [dev] of the
 * call's src_dtype, numel elements; first != 0 overwrites dst.
 * tile_sumsq / tile_flag [dev, optional, both or neither]: one slot per
 * MS_ACCUM_TILE elements of dst (ceil(numel / MS_ACCUM_TILE) slots); K5
 * writes each tile's fp64 sum of squares of the NEW dst values, unscaled
 * as ms_grad_stats unscales (the call's unscale / grad_scale), and a flag
 * that is non-zero iff one of those values is inf/nan (tested before
 * unscaling). */
typedef struct ms_accum_row {
  float* dst;
  const void* src;
  int64_t numel;
  int32_t first;
  int32_t reserved;     /* 0 */
  double* tile_sumsq;
  uint32_t* tile_flag;
} ms_accum_row_t;       /* 48 bytes */

/* Rows per K5 launch of ms_accumulate_grads (they travel in the kernel
 * arguments, so a batch needs no device-side table), and the elements one
 * K5 tile (one statistics slot) covers. */
#define MS_ACCUM_ROWS_PER_LAUNCH 64
#define MS_ACCUM_TILE 2048

/*
 * K5, batched: ms_accumulate_grad for every row of rows[0 .. nrows) [host
 * memory, read before the call returns], ceil(nrows / 64) launches.  Rows
 * with numel 0 are skipped; the dst ranges of one call must not overlap.
 * The contiguous-gradient hooks queue the gradients backward produces and
 * flush them through this call (at the end of backward, or when a bucket
 * fills), in place of one launch per parameter per micro-batch; same
 * reference lines as ms_accumulate_grad.  With tile statistics the same
 * pass also does the work of the boundary scan (K1) over the new sums:
 * the flag and per-tile sum of squares of flat.py:196-257 and
 * stage_1_and_2.py:105-116, which ms_reduce_tile_stats then folds into
 * ms_norm_clip's partial slots.  unscale: MS_SCALE_NONE or
 * MS_SCALE_DIVIDE (grad_scale > 0).
 */
int ms_accumulate_grads(const ms_accum_row_t* rows, int32_t nrows, int32_t src_dtype,
                        int32_t unscale, float grad_scale, void* stream);

/*
 * Fold per-tile statistics (K5's tile_sumsq / tile_flag of one group,
 * ntiles slots [dev]) into the nblk >= ms_stats_blocks() partial slots
 * ms_norm_clip reads for that group [dev]: slot j holds the fp64 sum of
 * tiles [j*ntiles/nblk, (j+1)*ntiles/nblk) in a fixed order (64 strided
 * partial sums added by a fixed tree) and the OR of their flags, so the
 * norm is a pure function of the tile statistics.
 * Replaces K1 (ms_grad_stats) at a contiguous-gradient boundary.
 */
int ms_reduce_tile_stats(const double* tile_sumsq, const uint32_t* tile_flag, int64_t ntiles,
                         double* block_sumsq, uint32_t* block_flag, int32_t nblk,
                         void* stream);

/* One group's part of ms_boundary_scalars_noalloc: the arguments
 * ms_grad_stats takes for it. */
typedef struct ms_group_scan {
  const ms_segment_t* segs; /* [dev] tiles [begin, end); may be NULL if empty */
  int32_t nseg;
  int32_t grad_dtype;       /* MS_DTYPE_* of segs[].grad */
  int64_t begin, end;       /* scanned flat range (flag) */
  int64_t own_begin, own_end; /* counted range (sum of squares) */
} ms_group_scan_t;

/*
 * K1 over every group, then K2: the boundary's scalars with no workspace
 * argument and no allocation.  No counterpart in minispeed; for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  Equals ms_grad_stats on each
 * group (block_sumsq / block_flag of group g at slot g * ms_stats_blocks())
 * followed by ms_norm_clip, bit for bit.
 *
 * groups [host]: ngroups entries, 0 <= ngroups <= MS_SCRATCH_MAX_GROUPS,
 *   each of at most MS_SCRATCH_MAX_TILES tiles (ceil((end - begin) /
 *   MS_SCAN_TILE); more: MS_ESCRATCH, nothing launched).  unscale /
 *   grad_scale apply to every group as in ms_grad_stats; the clip, scaler,
 *   out and out_host arguments are ms_norm_clip's.
 * The tile and partial slots live in a static device array of the library
 * (MS_SCRATCH_MAX_GROUPS x ms_stats_blocks() + MS_SCRATCH_MAX_TILES slots
 * of 12 bytes = 25.5 MiB), one per GPU, held until the process ends; its
 * address is looked up once per device on the first call there.  The groups
 * are scanned one after another through the same tile slots.  K1 writes
 * every tile slot the fold reads and the fold every slot K2 reads, so
 * nothing must be cleared between calls.  Calls that overlap on one GPU (two streams,
 * or two threads) share that array and race: serialize them.
 */
int ms_boundary_scalars_noalloc(const ms_group_scan_t* groups, int32_t ngroups,
                                int32_t unscale, float grad_scale, int32_t has_clip,
                                double max_norm, int32_t scaler_enabled, double scale,
                                int64_t good_steps, int64_t skipped_steps, int64_t window,
                                double min_scale, double max_scale, ms_step_scalars_t* out,
                                ms_step_scalars_t* out_host, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MINISPEED_BOUNDARY_H */

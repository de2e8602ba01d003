/*
 * luma.h -- C ABI of the MI355X (gfx950) LUMA optimizer-step library
 * (libluma_hip.so).  Plain C types only; every pointer documented as
 * "device" is HIP device memory owned by the caller.  The library never
 * allocates, never synchronises the stream it is given, and never throws:
 * each entry point returns 0 on success or a nonzero status whose text is
 * available from luma_last_error().
 *
 * Every per-step quantity lives in device memory: each tensor's step count,
 * scales and grids sit in its slot, and the step-dependent scalars are
 * derived on the device from the param group's hyper-parameters.  A launch
 * sequence captured into a HIP graph therefore advances correctly on every
 * replay (the reference keeps its step counter on the device for the same
 * reason, optimizer.py:382-387).
 *
 * What each entry point replaces in the reference (IgorYashch/LUMA 0.1.0):
 *
 *   luma_step          -- the per-parameter loop body of LUMA.step for all
 *                         parameters at once: luma_init_step (t = 1,
 *                         src/luma_optimizer/functional.py:183-228) and
 *                         luma_update_step (t >= 2, functional.py:231-298),
 *                         i.e. the Triton pipelines luma_triton_init_step /
 *                         luma_triton_step (triton_kernel.py:409-492); with
 *                         LumaScaling, also GradScaler's unscale_ and
 *                         skip-on-overflow around it (the reference runs
 *                         them outside the optimizer).
 *   luma_step_profiled -- luma_step with event records between its launches.
 *   luma_step_noalloc  -- luma_step with its workspace inside the library
 *                         (no counterpart in the reference; for callers that
 *                         cannot allocate).
 *   luma_step_tensor   -- one tensor, no device tables: the per-tensor
 *                         functional ops luma_triton_step /
 *                         luma_triton_init_step (triton_kernel.py:409-492).
 *   luma_set_scales    -- the scale half of load_state_dict /
 *                         _init_triton_buffers (optimizer.py:146-183,341-387).
 *   luma_get_scales    -- the S_m / S_v / step read-back of state_dict
 *                         (optimizer.py:119-144).
 *   luma_decode        -- the decode of export_adamw_state
 *                         (optimizer.py:231-235, functional.py:113-126).
 *   luma_quantize      -- the quantisation of import_adamw_state
 *                         (optimizer.py:304-321, functional.py:133-176).
 *   luma_hyper_rows    -- the step-dependent scalars of functional.py:209-213,
 *                         262-264, 278 as the device derives them (for
 *                         checking against the host's double arithmetic).
 *   luma_philox4x32    -- host-side Philox4x32-10 block function used by the
 *                         stochastic rounding (Salmon et al., SC'11); the
 *                         reference's Triton path draws from tl.rand
 *                         (triton_kernel.py:103,124).
 */
#ifndef LUMA_H
#define LUMA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LUMA_ABI_VERSION 9

/*
 * Elements per chunk-table entry (one workgroup's share of a tensor): the
 * default and the largest.  luma_step accepts any power of two from
 * LUMA_CHUNK_ELEMS_MIN to LUMA_CHUNK_ELEMS per launch (LumaStepArgs.chunk_elems);
 * smaller chunks give small tensor sets more workgroups.
 */
#define LUMA_CHUNK_ELEMS 131072
#define LUMA_CHUNK_ELEMS_MIN 2048
#define LUMA_STEP_TENSOR_CHUNK_MIN 16384   /* shortest chunk luma_step_tensor uses */

/*
 * Tensors of at most this many elements are best stepped one wavefront each
 * with an exact pass 1 (LumaStepArgs.small_chunks): a workgroup of their own
 * would spend most of its time in set-up, and the fast pass 1's wavefront
 * route (medium_chunks) runs a partial group for them.
 */
#define LUMA_SMALL_TENSOR 256

/*
 * Tensors above LUMA_SMALL_TENSOR and of at most this many elements are best
 * stepped one wavefront each (LumaStepArgs.medium_chunks): a whole
 * workgroup would leave most of its wavefronts idle on them.
 */
#define LUMA_MEDIUM_TENSOR 8192

/*
 * Bytes of one slot: a tensor's persistent device state (step count, S_m,
 * S_v, grids).  A fresh slot must be zero-filled (step count 0: the next
 * step is the reference's init step).  16-byte aligned.
 */
#define LUMA_SLOT_BYTES 512

/*
 * Code summaries.  A tensor may carry a summary array that its steps keep:
 * one uint32 per thread of each chunk's workgroup, LUMA_SUMMARY_WORDS words
 * per chunk, chunk c of the tensor at words [c * LUMA_SUMMARY_WORDS,
 * (c + 1) * LUMA_SUMMARY_WORDS).  Each step's pass 2 writes, for every
 * thread, a bound on the codes it stored in its share of the chunk: the
 * largest |Q_m| and the smallest Q_w, widened by the step's certified
 * decision margin.  The next step's pass 1 bounds each thread's |m'| and v'
 * from that word and the gradients alone, and reads a wave's codes only when
 * some thread could hold the tensor's maximum.  Results do not depend on the
 * summaries; they only save reads.  They are used only when the slot records
 * that the previous step wrote them with the same chunk length (luma_set_scales
 * and luma_quantize clear that record), and only for chunks whose words fit
 * in summary_words.  A caller that rewrites a tensor's codes by other means
 * between steps must also rewrite its slot with luma_set_scales, or pass a
 * NULL summary.  luma_summary_words gives the words a tensor needs.
 */
#define LUMA_SUMMARY_WORDS 256

/* Gradient element types. */
#define LUMA_GRAD_F32 0
#define LUMA_GRAD_BF16 1
#define LUMA_GRAD_F16 2

/*
 * Where the stochastic-rounding uniforms come from.  Under
 * LUMA_NOISE_INJECTED a tensor whose u_m or u_w is NULL draws from Philox as
 * under LUMA_NOISE_PHILOX, so a caller may inject uniforms for some tensors
 * of a step only.
 */
#define LUMA_NOISE_PHILOX 0   /* counter-based Philox4x32-10, keyed per (seed, step, param) */
#define LUMA_NOISE_INJECTED 1 /* caller-supplied u_m / u_w float32 arrays in [0, 1) */

/* luma_step flags. */
#define LUMA_FLAG_EXACT_ONLY 1 /* take the exact per-element path everywhere */

/* One parameter tensor taking part in a step. */
typedef struct LumaTensor {
  float *param;         /* device f32 [numel], updated in place            */
  const void *grad;     /* device f32 / bf16 / f16 [numel]                  */
  int16_t *q_m;         /* device [numel] signed log-grid momentum codes    */
  int16_t *q_w;         /* device [numel] uint16 preconditioner codes       */
  const float *u_m;     /* device [numel] injected uniforms, or NULL        */
  const float *u_w;     /* device [numel] injected uniforms, or NULL        */
  void *slot;           /* device, LUMA_SLOT_BYTES: this tensor's state     */
  uint32_t *summary;    /* device code summaries kept across steps, or NULL */
  int64_t summary_words;/* words at summary (see luma_summary_words)       */
  int64_t numel;        /* elements                                          */
  int64_t param_id;     /* position of the parameter in param_groups order  */
  int64_t elem_offset;  /* index of element 0 in the whole parameter when this
                           tensor is one shard of it, else 0: the Philox
                           counters follow the whole parameter's element
                           index, so shards draw independent uniforms       */
  int32_t grad_dtype;   /* LUMA_GRAD_*                                       */
  int32_t group;        /* index into the LumaGroup table                    */
  int32_t first_chunk;  /* index of this tensor's first LumaChunk            */
  int32_t reserved;     /* 0                                                 */
} LumaTensor;

/* Chunk c of a tensor covers elements [c*C, min(numel, (c+1)*C)), C the launch's chunk length. */
typedef struct LumaChunk {
  int32_t tensor; /* index into the LumaTensor table */
  int32_t index;  /* chunk number within that tensor */
} LumaChunk;

/*
 * A param group's hyper-parameters as the Python doubles the reference holds
 * (optimizer.py:80-92).  Per step the device derives, exactly as the
 * reference's double arithmetic and each rounded once to float32:
 * beta1, 1 - beta1, beta2, 1 - beta2, 1 - weight_decay*lr,
 * -(lr / (1 - beta1^t)), 1 - beta2^t and eps, where beta^t is the correctly
 * rounded power (Python's ** agrees with it after the float32 rounding).
 */
typedef struct LumaGroup {
  double lr, beta1, beta2, eps, weight_decay;
  double reserved; /* 0 */
} LumaGroup;

/*
 * Mixed-precision scaling (torch.amp.GradScaler's contract for optimizers
 * that unscale inside their step, `_step_supports_amp_scaling`):
 *   grad_scale -- device float32 scalar, or NULL.  The gradients hold
 *                 scale * g; each element is unscaled exactly as
 *                 GradScaler.unscale_ would store it:
 *                 dtype(f32(grad) * f32(1 / (double)scale)), rounded to
 *                 nearest even in the gradient's own dtype.
 *   found_inf  -- device float32 scalar, or NULL.  Nonzero: the whole step
 *                 does nothing (parameters, codes, scales and step counts
 *                 unchanged), with no host synchronisation.
 */
typedef struct LumaScaling {
  const float *grad_scale;
  const float *found_inf;
} LumaScaling;

typedef struct LumaStepArgs {
  const LumaTensor *tensors; /* device */
  int32_t n_tensors;
  int32_t n_chunks;
  const LumaChunk *chunks;   /* device */
  const LumaGroup *groups;   /* device */
  float *partials;           /* device workspace, luma_workspace_bytes(n_chunks), 16-byte aligned */
  uint64_t base_seed;        /* LUMA._base_seed as its two's-complement bits */
  int32_t noise_mode;        /* LUMA_NOISE_* */
  int32_t flags;             /* LUMA_FLAG_* */
  int32_t chunk_elems;       /* chunk length C of the chunk table: a power of two in
                                [LUMA_CHUNK_ELEMS_MIN, LUMA_CHUNK_ELEMS]; 0 = LUMA_CHUNK_ELEMS */
  int32_t small_chunks;      /* the last small_chunks records of the chunk table, one
                                chunk per tensor, are stepped one wavefront each (four
                                per workgroup): pass 1 by the exact path, pass 2 by the
                                fast kernel's wavefront route; meant for tensors of at
                                most LUMA_SMALL_TENSOR elements (any tensor is stepped
                                correctly).  0: every chunk takes a workgroup */
  int32_t medium_chunks;     /* the medium_chunks records just before the small ones
                                are stepped one wavefront each, four per workgroup, in
                                the same launches and by the same fast kernels as the
                                others (8 elements per lane and iteration); meant for
                                tensors of at most LUMA_MEDIUM_TENSOR elements, one
                                chunk each (any chunk is stepped correctly).  Such
                                tensors keep no code summaries.  0: none */
  int32_t reserved;          /* 0 */
  LumaScaling scaling;       /* both NULL: unscaled gradients, always step */
} LumaStepArgs;

/* One slot write (array in device memory). */
typedef struct LumaScaleInit {
  void *slot;    /* device slot */
  int64_t step;  /* the tensor's step count t */
  double s_m;    /* S_m as stored by the reference (>= 1e-9) */
  double s_v;    /* S_v (>= 0) */
  double eps;    /* the group's eps */
} LumaScaleInit;

int luma_abi_version(void);
const char *luma_last_error(void);

/*
 * Struct sizes as compiled, for binding checks: LumaTensor, LumaChunk,
 * LumaGroup, LumaScaleInit, LumaStepArgs, slot bytes, LUMA_CHUNK_ELEMS, 0.
 */
void luma_layout(int32_t out[8]);

/* Bytes of workspace luma_step / luma_step_tensor / luma_quantize need for n_chunks chunks. */
size_t luma_workspace_bytes(int32_t n_chunks);

/* Summary words a tensor of numel elements needs for chunks of chunk_elems elements. */
int64_t luma_summary_words(int64_t numel, int32_t chunk_elems);

/*
 * One optimizer step for every tensor in the table: pass 1 (decode + EMA +
 * per-chunk maxima), per-tensor finalize (new S_m/S_v and grid in float64,
 * step count + 1, step scalars), pass 2 (re-decode + EMA + AdamW update +
 * LogSR re-quantisation).  A tensor whose slot holds step count 0 takes the
 * init step.  Three kernel launches on `stream` (a hipStream_t): the small
 * tensors (small_chunks > 0) are stepped by workgroups of the pass-1 and
 * pass-2 launches past their own (with LUMA_FLAG_EXACT_ONLY by a kernel of
 * their own in each pass); no host synchronisation.  No device table is written, so the sequence may
 * be captured into a HIP graph and replayed.
 */
int luma_step(const LumaStepArgs *args, void *stream);

/*
 * luma_step that also records caller-created hipEvent_t events[0..3] on the
 * stream: before pass 1, after pass 1, after finalize, after pass 2 (NULL
 * entries are skipped).  Used to time each kernel on its own stream.
 */
int luma_step_profiled(const LumaStepArgs *args, void *stream, void *const events[4]);

/*
 * Largest n_chunks luma_step_noalloc takes: its workspace is a fixed device
 * array of 16 bytes per chunk (4 MiB per GPU).
 */
#define LUMA_NOALLOC_MAX_CHUNKS 262144

/*
 * luma_step that allocates nothing and takes no workspace: args->partials is
 * ignored, and pass 1's per-chunk maxima go to a fixed array inside the
 * library (one per GPU, kept until the process ends), so no memory is
 * allocated on any call, the first included.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Limits:
 * n_chunks <= LUMA_NOALLOC_MAX_CHUNKS (else an error, nothing launched); the
 * stream's device must be the current device; calls that overlap on one GPU
 * (other streams, other threads) share that GPU's array and race.
 */
int luma_step_noalloc(const LumaStepArgs *args, void *stream);

/*
 * luma_step for one tensor with no device tables: *tensor, *group and
 * *scaling (may be NULL) are host structs read during the call
 * (tensor->first_chunk is ignored).  The chunk length is LUMA_CHUNK_ELEMS,
 * halved down to LUMA_STEP_TENSOR_CHUNK_MIN while the tensor has fewer than
 * 4096 chunks; `partials` needs
 * luma_workspace_bytes(ceil(numel / LUMA_STEP_TENSOR_CHUNK_MIN)).
 */
int luma_step_tensor(const LumaTensor *tensor, const LumaGroup *group, float *partials,
                     uint64_t base_seed, int32_t noise_mode, int32_t flags,
                     const LumaScaling *scaling, void *stream);

/* Write step count, S_m and S_v of n slots (items: device array) and derive their grids. */
int luma_set_scales(const LumaScaleInit *items, int32_t n, void *stream);

/*
 * Read n slots (slots: device array of slot pointers): S_m, S_v into
 * scales[2*i], scales[2*i+1] and the step count into steps[i] (device).
 */
int luma_get_scales(void *const *slots, int32_t n, double *scales, int64_t *steps, void *stream);

/*
 * Decode one tensor's codes into float32 m (exp_avg) and v (exp_avg_sq) on
 * the grid of the slot's current step, with the group's eps.
 */
int luma_decode(const int16_t *q_m, const int16_t *q_w, int64_t numel, const void *slot,
                double eps, float *m_out, float *v_out, void *stream);

/*
 * Quantise given float32 m, v (clamped at 0) into codes with fresh scales
 * S_m = max(max|m|, 1e-9), S_v = max(max v, 0), stored into the slot with
 * step count `step`.  Uniforms: Philox keyed by seed (noise_mode 0) or
 * u_m/u_w (noise_mode 1).  `partials` needs
 * luma_workspace_bytes(ceil(numel / LUMA_CHUNK_ELEMS)).
 */
int luma_quantize(const float *m, const float *v, int64_t numel, int16_t *q_m, int16_t *q_w,
                  void *slot, int64_t step, double eps, uint64_t seed, int32_t noise_mode,
                  const float *u_m, const float *u_w, float *partials, void *stream);

/*
 * The step scalars the device derives for steps t0 .. t0+n-1 of *group (a
 * host struct): 8 floats per step into out (device): beta1, 1-beta1, beta2,
 * 1-beta2, decay, -eta, bc2, eps.
 */
int luma_hyper_rows(const LumaGroup *group, int64_t t0, int32_t n, float *out, void *stream);

/* Host: one Philox4x32-10 block. */
void luma_philox4x32(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

#ifdef __cplusplus
}
#endif

#endif /* LUMA_H */

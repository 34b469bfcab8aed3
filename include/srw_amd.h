/*
 * srw_amd.h -- C ABI of the MI355X-native Select-Read-Write (SRW) unit-pool
 * layer (DAWN-SRW v4.1 / v4.0.1 gate), built for gfx950.
 *
 * One call computes, for every token t and route r of a pool of N rank-1
 * units with rows e_n (routing, d_route), r_n (read, d_model) and w_n
 * (write, d_model):
 *
 *   s[t,n]   = h[t,r,:] . e_n                         (score)
 *   tau[t]   = mean_n s + tau_offset[t,r] * (std_n s + 1e-8)
 *   gate     = sigmoid(k (s - tau - a)) * (eps + min(max(s - tau - a - c, 0), M))   (v4.1)
 *            | z Phi(z), z = (s - tau)/std, 0 for z <= 0                          (v4.0.1)
 *   out[t,r] = scale * sum_n gate * (x[t,:] . r_n) * w_n / max(den, 1)
 *   den      = sum_n intensity (v4.1) | sum_n gate (v4.0.1)
 *
 * Reference interfaces replaced (paths relative to madst0614/DAWN-SRW):
 *   srw_forward, n_routes = 1, SRW_STATS_ONEPASS
 *       -> make_sharded_srw(...) -> fused_gate_srw(x, h, emb, tau_offset,
 *          read, write)                models/dawn_spatial_v41_exp.py:352-637
 *   srw_forward, n_routes = 2, SRW_STATS_ONEPASS
 *       -> make_sharded_srw_paired(...) -> fused_gate_srw_paired(...)
 *                                         models/dawn_spatial_v41_exp.py:640-909
 *   srw_forward, n_routes = 1, SRW_STATS_CENTERED, dtype = SRW_F32
 *       -> _srw_inference(x, h, emb_norm, tau_offset, w_read, w_write)
 *                                         models/dawn_spatial_v41_exp.py:1713-1738
 *   gate = SRW_GATE_GELU_V401
 *       -> fused_gate_srw / _srw_inference of
 *          models/legacy/dawn_spatial_v401_exp.py:229-355, 1443-1463
 *   srw_backward, n_routes = 1, SRW_STATS_ONEPASS, dtype = SRW_BF16
 *       -> the VJP of fused_gate_srw that jax.value_and_grad(loss_fn) takes in
 *          train_step (scripts/train_jax.py:548-726, through the sharded_fns
 *          tuple of :2324-2333): cotangents of out, score_lb and
 *          dead_penalty (the outputs the loss uses, :586-603) in, gradients of
 *          x, h, emb, tau_offset, read and write out; with gate =
 *          SRW_GATE_GELU_V401 the VJP of the v4.0.1 fused function
 *          (models/legacy/dawn_spatial_v401_exp.py:229-554: out and score_lb,
 *          the lb_loss of its callers, :978)
 *   srw_forward, dtype = SRW_F32, SRW_STATS_ONEPASS
 *       -> no reference counterpart (an extension: the reference's
 *          fused_gate_srw casts every operand to bf16, v41:422-428); checked
 *          against this library's scalar kernels only (parity unpinned)
 *   the closure constants of the factories (v41:297-301, 352-383) travel in
 *   srw_desc_t; srw_desc_init() fills the reference defaults.
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller; row-major,
 *     contiguous.  The library calls no allocator: scratch memory is the
 *     caller's workspace (size from srw_workspace_size), or, for
 *     srw_forward_noalloc, a static per-GPU array inside the library.
 *   - x, h, emb, read, write and out share desc->dtype (SRW_BF16 or SRW_F32).
 *     tau_offset and every per-token / per-unit statistic are float32.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *     is asynchronous.  srw_forward keeps no state between calls beyond the
 *     caller's workspace and is thread-safe; calls that share a workspace
 *     must not overlap (srw_forward_noalloc: every call on one GPU shares
 *     its scratch).
 *   - Errors are status codes; no C++ exception crosses the ABI.  NaN / Inf
 *     inputs propagate as in the reference (no extra clamping).
 */
#ifndef SRW_AMD_H
#define SRW_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SRW_AMD_ABI_VERSION 7

typedef enum srw_status {
  SRW_OK = 0,
  SRW_EINVAL = 1,       /* bad shape, pointer or constant */
  SRW_EUNSUPPORTED = 2, /* valid request the library does not implement */
  SRW_EHIP = 3,         /* a HIP runtime call failed (launch, device query) */
  SRW_EWORKSPACE = 4,   /* workspace missing or smaller than required */
  SRW_ESCRATCH = 5      /* srw_forward_noalloc: the call needs more than its scratch */
} srw_status_t;

typedef enum srw_dtype {
  SRW_F32 = 0,
  SRW_BF16 = 1
} srw_dtype_t;

typedef enum srw_gate {
  SRW_GATE_V41 = 0,       /* activation x intensity (v41:505-511) */
  SRW_GATE_GELU_V401 = 1  /* z Phi(z), R/W rows forward-normalised (v401:294-310) */
} srw_gate_t;

typedef enum srw_stats_mode {
  /* One-pass moments of the dtype-rounded scores: s_std = sqrt(E[s^2] -
   * mean^2) + 1e-8 (fused_gate_srw pass 1, v41:433-464). */
  SRW_STATS_ONEPASS = 0,
  /* Two-pass centred variance: s_std = sqrt(E[(s-mean)^2]) + 1e-8
   * (_srw_inference, v41:1717-1722). */
  SRW_STATS_CENTERED = 1,
  /* Closed form: sum s = h.(sum e), sum s^2 = h^T (E^T E) h.  Skips the
   * score pre-pass; moments come from unrounded scores. */
  SRW_STATS_GRAM = 2
} srw_stats_mode_t;

/* desc->flags */
#define SRW_FLAG_DIAG 0x1u        /* fill token_diag / unit_diag (training diagnostics) */
#define SRW_FLAG_EMULATE 0x2u     /* reference rounding emulation (per-chunk bf16 rounding
                                     of the partial write GEMM, v41:518); selects the
                                     bit-faithful scalar kernels */
#define SRW_FLAG_SPARSE_SKIP 0x4u /* skip units no row passes: the decode kernel (calls of
                                     <= 128 rows) leaves out the read rows and write-fragment
                                     halves of units no row of the call passes; the tiled
                                     family (d_model 256 / 512 / 1024) runs the read and
                                     write GEMMs of each 32-row tile over the units some row
                                     of the tile passes.  Exact for the v4.0.1 gate (their
                                     gates are 0); under v4.1 their epsilon-sized gates are
                                     left out of out only (sums, den and the mask keep
                                     them).  Other paths run dense (no counterpart in the
                                     reference, which computes every unit). */
#define SRW_FLAG_NO_FAST 0x8u     /* force the generic kernels (testing) */
#define SRW_FLAG_POOL_CACHED 0x10u /* emb, read and write are unchanged since the last call
                                      that used this workspace with the same descriptor:
                                      reuse the packed W^T and Gram statistics kept in the
                                      workspace (decode steps, layers sharing one pool).
                                      No counterpart in the reference, which recasts its
                                      pools on every call (v41:423-430). */
#define SRW_FLAG_TILED 0x20u      /* run the tiled-GEMM kernels (gated product P materialised
                                     in the workspace as bf16) even where a fused kernel
                                     exists; without the flag they serve bf16 shapes the
                                     fused kernels do not (d_model > 384, e.g. 1024 / 1280 /
                                     2048; both widths multiples of 64).  No counterpart in
                                     the reference (a kernel-family choice). */
#define SRW_FLAG_GATE_OUT 0x40u   /* the call passes outputs->gate: the workspace query and
                                     the kernel choice take the tiled matrix-core families
                                     (bf16 d_model / d_route multiples of 64, fp32 multiples
                                     of 32; v4.1, one-pass or centred statistics), whose
                                     gate epilogue also writes every unit's fp32 gate.
                                     Without it a gate output runs the generic kernels. */

typedef struct srw_desc {
  int64_t T;          /* tokens (B*S) */
  int64_t d_model;    /* D: x, read, write, out rows */
  int64_t d_route;    /* dr: h, emb rows */
  int64_t n_units;    /* N: pool rows */
  int32_t n_routes;   /* 1 = single route, 2 = paired (QK) sharing one x.R^T */
  int32_t dtype;      /* srw_dtype_t */
  int32_t gate;       /* srw_gate_t */
  int32_t stats_mode; /* srw_stats_mode_t */
  float sharpness;        /* v4.1 SHARPNESS            (default 500)  */
  float act_threshold;    /* v4.1 ACTIVATION_THRESHOLD (default 0.5)  */
  float act_cutoff;       /* v4.1 ACTIVATION_CUTOFF    (default 0.01) */
  float epsilon;          /* v4.1 EPSILON              (default 1e-4) */
  float max_intensity;    /* v4.1 MAX_INTENSITY        (default 10)   */
  float dead_threshold;   /* dead-unit threshold for unit_diag consumers (0.01) */
  float scale;            /* multiplies out after the den division (1 = reference fn) */
  int32_t chunk_size;     /* N-chunk of the reference plan (v41:416-420); 0 = one
                             chunk.  The matrix-core and tiled kernels round each
                             chunk's partial write GEMM to bf16 before the chunks
                             are summed (v41:518, the chunk scan :489-577) and
                             never let an N-split cross a chunk; the generic
                             kernels do so under SRW_FLAG_EMULATE */
  uint32_t flags;         /* SRW_FLAG_* */
  int32_t reserved[3];
} srw_desc_t;

/* Per-token diagnostics, token_diag[(t * n_routes + r) * SRW_TDIAG_COUNT + k]. */
enum {
  SRW_TDIAG_S_MEAN = 0,   /* mean_n s */
  SRW_TDIAG_S_STD,        /* std_n s + 1e-8 */
  SRW_TDIAG_TAU,          /* tau */
  SRW_TDIAG_SUM_S3,       /* sum_n s^3 (ONEPASS mode; 0 otherwise) */
  SRW_TDIAG_SUM_S4,       /* sum_n s^4 (ONEPASS mode; 0 otherwise) */
  SRW_TDIAG_GATE_MAX,     /* max_n gate */
  SRW_TDIAG_INT_SUM,      /* sum_n intensity (v4.1) | sum_n z+ (v4.0.1), before the floor */
  SRW_TDIAG_N_STRONG,     /* #act > 0.9  (v4.0.1: #gate > 0.5) */
  SRW_TDIAG_N_BOUNDARY,   /* #0.1 < act < 0.9 (v4.0.1: #phi > .95 or phi < .05) */
  SRW_TDIAG_N_BAND075,    /* #0.05 < act < 0.95 (v4.0.1: #0 < z < 0.75) */
  SRW_TDIAG_N_BAND030,    /* #0.2 < act < 0.8 (v4.0.1: #0 < z < 0.30) */
  SRW_TDIAG_G_LOG_G,      /* sum_n gate * log(gate + 1e-8) */
  SRW_TDIAG_INT_MAX,      /* max_n intensity (v4.0.1: 0) */
  SRW_TDIAG_N_INT_CAP,    /* #intensity >= eps + max_intensity - 1e-3 (v4.0.1: 0) */
  SRW_TDIAG_COUNT
};

/* Per-unit diagnostics, unit_diag[n * SRW_UDIAG_COUNT + k]; reduced over all
 * tokens and routes of the call (v41:543-552, 445-447). */
enum {
  SRW_UDIAG_SCORE_SUM = 0, /* sum_{t,r} s[t,r,n] */
  SRW_UDIAG_GATE_MAX,      /* max_{t,r} gate[t,r,n] */
  SRW_UDIAG_COUNT
};

typedef struct srw_tensors {
  const void* x;           /* [T, D] */
  const void* h;           /* [T, n_routes, dr]; may alias x when n_routes == 1, dr == D */
  const void* emb;         /* [N, dr] */
  const float* tau_offset; /* [T, n_routes] */
  const void* read;        /* [N, D] */
  const void* write;       /* [N, D] */
} srw_tensors_t;

typedef struct srw_outputs {
  void* out;               /* [T, n_routes, D] (required) */
  float* gate_sum;         /* [T, n_routes]   sum_n gate            (optional) */
  float* den;              /* [T, n_routes]   max(den, 1)           (optional) */
  int32_t* n_active;       /* [T, n_routes]   #units with act > 0.5 (optional) */
  uint64_t* pass_mask;     /* [T, n_routes, ceil(N/64)] bit n%64 of word n/64 set
                              iff unit n passes (act > 0.5)        (optional) */
  float* token_diag;       /* [T, n_routes, SRW_TDIAG_COUNT]  needs SRW_FLAG_DIAG */
  float* unit_diag;        /* [N, SRW_UDIAG_COUNT]            needs SRW_FLAG_DIAG */
  float* gate;             /* [T, n_routes, N] gate (activation x intensity, fp32) of every
                              unit: the gate_raw of _srw_inference_with_gates
                              (models/dawn_spatial_v41_exp.py:1741-1769).  Optional; with
                              SRW_FLAG_GATE_OUT the tiled families write it, else the
                              call runs the generic kernels. */
} srw_outputs_t;

/* Cotangents for srw_backward: of the three outputs of fused_gate_srw that
 * enter the reference's training loss (scripts/train_jax.py:586-603). */
typedef struct srw_cotangents {
  const float* d_out;      /* [T, n_routes, D] cotangent of out (required) */
  const void* out;         /* [T, n_routes, D] out of the forward call on the same
                              inputs (desc->dtype; required: the den term) */
  float d_score_lb;        /* cotangent of score_lb (v41:477-483) */
  float d_dead_penalty;    /* cotangent of dead_penalty (v41:543-552) */
  /* Optional residuals of that forward call, both or neither: its den and
   * its unit_diag (a call with SRW_FLAG_DIAG, as the drop-in's forward
   * makes).  With them the backward takes den, each unit's mean score
   * (score_lb) and max gate (the dead units) from the forward instead of
   * recomputing them in a pass of its own over the scores (no counterpart
   * in the reference, whose autodiff keeps its own residuals; values equal
   * up to the forward's summation order). */
  const float* den;        /* [T, n_routes] or NULL */
  const float* unit_diag;  /* [N, SRW_UDIAG_COUNT] or NULL */
} srw_cotangents_t;

/* Gradients written by srw_backward, float32; all required but dscale.
 * When the forward's h was x itself (d_route == d_model), the gradient of x
 * is dx + dh (the two paths are returned separately). */
typedef struct srw_grads {
  float* dx;               /* [T, D] */
  float* dh;               /* [T, n_routes, d_route] */
  float* demb;             /* [N, d_route] */
  float* dtau_offset;      /* [T, n_routes] */
  float* dread;            /* [N, D] */
  float* dwrite;           /* [N, D] */
  float* dscale;           /* [1] gradient of desc->scale: sum d_out * out / scale,
                              the gradient of the caller's *_scale multiply
                              (v41:1044-1053, 1175); optional (NULL: skipped) */
} srw_grads_t;

/* ABI version of the loaded library (SRW_AMD_ABI_VERSION). */
int32_t srw_abi_version(void);

/* Human-readable name of a status code (static storage). */
const char* srw_status_string(srw_status_t status);

/* Fill *desc with the v4.1 reference defaults (v41:297-301, 352; scale 1,
 * SRW_BF16, SRW_GATE_V41, SRW_STATS_ONEPASS, n_routes 1, chunk_size 0) and
 * zero shapes. */
srw_status_t srw_desc_init(srw_desc_t* desc);

/* Validate *desc and report the workspace (device bytes) srw_forward needs:
 * the larger of the kernel families the call may take (with d_route ==
 * d_model and one route, passing h == x can select a different family). */
srw_status_t srw_workspace_size(const srw_desc_t* desc, size_t* bytes);

/* Enqueue one SRW layer forward on `stream`.  Replaces fused_gate_srw /
 * fused_gate_srw_paired / _srw_inference (see the table at the top). */
srw_status_t srw_forward(const srw_desc_t* desc, const srw_tensors_t* in,
                         const srw_outputs_t* outs, void* workspace,
                         size_t workspace_bytes, void* stream);

/* srw_forward without a workspace argument and without allocating.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  The workspace is a static scratch array of
 * SRW_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held from the
 * library's first use on that GPU until the process ends; its device address
 * is looked up once per device.  The same kernels run as in srw_forward, so
 * the results are equal bit for bit.  Limits: a call whose
 * srw_workspace_size exceeds the scratch returns SRW_ESCRATCH with nothing
 * launched (64 MiB holds every decode-sized call of the 40M pools up to 128
 * rows; prefill-sized calls need srw_forward); SRW_FLAG_POOL_CACHED is
 * refused (SRW_EINVAL), since the scratch keeps whatever the last call on that
 * GPU left in it.  All calls on one GPU share its scratch: calls that overlap
 * on one GPU (two streams, two threads) race -- serialise them. */
#define SRW_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
srw_status_t srw_forward_noalloc(const srw_desc_t* desc, const srw_tensors_t* in,
                                 const srw_outputs_t* outs, void* stream);

/* Several independent srw_forward calls on one stream.  No counterpart in
 * the reference, whose layer issues each pool's SRW as a call of its own
 * (the Q, K and V projections, v41:1784-1799 in the KV-cache step and
 * :1036-1053 in the forward): equivalent to srw_forward(&descs[i], &ins[i],
 * &outs[i], ws_i, bytes_i, stream) for i = 0 .. n-1 in order, where ws_i is
 * call i's slice of `workspace` (srw_workspace_size_batch), with equal
 * results bit for bit.  Calls on the matrix-core kernels (bf16, no
 * diagnostics, one-pass or centred statistics) with the same d_model,
 * d_route and statistics that take the same kernel instantiations -- all the
 * decode kernel (at most 128 rows), or all the same prefill main kernel --
 * run as one launch per stage (the small pools' calls are bound by their
 * launches); otherwise the calls run one after the other.  1 <= n <=
 * SRW_MAX_BATCH; the calls must not share outputs. */
#define SRW_MAX_BATCH 4
srw_status_t srw_workspace_size_batch(int32_t n, const srw_desc_t* descs, size_t* bytes);
srw_status_t srw_forward_batch(int32_t n, const srw_desc_t* descs, const srw_tensors_t* ins,
                               const srw_outputs_t* outs, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Validate *desc for srw_backward and report its workspace (device bytes). */
srw_status_t srw_backward_workspace_size(const srw_desc_t* desc, size_t* bytes);

/* Enqueue the reverse-mode derivative (VJP) of one srw_forward call on
 * `stream`: recomputes the forward's scores, gates and products from the
 * inputs (as the reference's jax.checkpoint-ed scans do, v41:434, 489) and
 * writes the gradients of <d_out, out> + d_score_lb * score_lb +
 * d_dead_penalty * dead_penalty.  bf16, the v4.1 gate or the v4.0.1 GELU
 * gate (whose function has no dead_penalty: d_dead_penalty must be 0, else
 * SRW_EINVAL; read and write enter through the forward normalisation), one
 * route or the paired routes (n_routes = 2, fused_gate_srw_paired),
 * one-pass statistics, d_model and d_route multiples of 64; anything else
 * returns SRW_EUNSUPPORTED.  Every tensor and gradient pointer 16-byte
 * aligned (as device allocations are), else SRW_EINVAL.  With
 * T = 0 the gradients of emb, read, write (and dscale) are zero.  The cotangents of bf16 values are rounded to bf16 where
 * the reference's bf16 casts, dots and products transpose (the gradients are
 * bf16 dot outputs widened to float32). */
srw_status_t srw_backward(const srw_desc_t* desc, const srw_tensors_t* in,
                          const srw_cotangents_t* cot, const srw_grads_t* grads,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Name of the kernel family the last srw_forward on this thread used
 * ("generic", "mfma_bf16", "mfma_ss_bf16", ...), for tests and benchmarks. */
const char* srw_last_path(void);

/* Profiling hook; no counterpart in the reference (its timing is host-side
 * time.time() around whole calls, scripts/train_jax.py:2469-2481).  When
 * both are non-NULL, every later srw_forward on this thread records the
 * hipEvent_t `start` on the call's stream right before its dominant kernel
 * (the fused score/read/gate/write kernel) and `stop` right after it, so a
 * benchmark can time that kernel alone.  NULL, NULL switches it off. */
srw_status_t srw_set_kernel_events(void* start, void* stop);

#ifdef __cplusplus
}
#endif

#endif /* SRW_AMD_H */

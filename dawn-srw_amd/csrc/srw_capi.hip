// srw_capi.hip -- the extern "C" boundary of libsrw_amd.so.
//
// Validates a call, sizes the workspace, picks a kernel family and enqueues
// it on the caller's stream.  No allocation; global state: the per-thread
// name of the last path taken and, for srw_forward_noalloc, the device
// address of the static scratch array per device.

#include <math.h>
#include <string.h>

#include <mutex>

#include "srw_internal.hpp"

// Workspace of srw_forward_noalloc: a static array in the library's code
// object, so each GPU the library runs on holds its own copy (at its own
// address) from the code object's load until the process ends.  Host code
// never passes the name `scratch` to a kernel or a copy -- on the host it
// names a shadow, not device memory -- but the device address that
// hipGetSymbolAddress returns for the current device (scratch_address).
static __device__ __align__(256) char scratch[SRW_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local const char* g_last_path = "none";
thread_local hipEvent_t g_ev_start = nullptr;
thread_local hipEvent_t g_ev_stop = nullptr;

srw_status_t validate(const srw_desc_t* d) {
  if (!d) return SRW_EINVAL;
  if (d->T < 0 || d->d_model < 1 || d->d_route < 1 || d->n_units < 1) return SRW_EINVAL;
  if (d->n_routes != 1 && d->n_routes != 2) return SRW_EINVAL;
  if (d->dtype != SRW_F32 && d->dtype != SRW_BF16) return SRW_EINVAL;
  if (d->gate != SRW_GATE_V41 && d->gate != SRW_GATE_GELU_V401) return SRW_EINVAL;
  if (d->stats_mode != SRW_STATS_ONEPASS && d->stats_mode != SRW_STATS_CENTERED &&
      d->stats_mode != SRW_STATS_GRAM)
    return SRW_EINVAL;
  if (d->chunk_size < 0) return SRW_EINVAL;
  if (!isfinite(d->sharpness) || !isfinite(d->act_threshold) || !isfinite(d->act_cutoff) ||
      !isfinite(d->epsilon) || !isfinite(d->max_intensity) || !isfinite(d->scale))
    return SRW_EINVAL;
  if (d->flags & ~(SRW_FLAG_DIAG | SRW_FLAG_EMULATE | SRW_FLAG_SPARSE_SKIP | SRW_FLAG_NO_FAST | SRW_FLAG_POOL_CACHED |
                   SRW_FLAG_TILED | SRW_FLAG_GATE_OUT))
    return SRW_EINVAL;
  return SRW_OK;
}

// Which family serves this descriptor: 1 = fused MFMA, 2 = tiled GEMMs,
// 3 = fp32 tiled GEMMs, 0 = generic, -1 = none.  h_is_x: h aliases x (known to srw_forward from
// the pointers).
int choose(const srw_desc_t& d, bool h_is_x) {
  const bool force_generic = (d.flags & (SRW_FLAG_EMULATE | SRW_FLAG_NO_FAST)) != 0;
  if (!force_generic && (d.flags & SRW_FLAG_GATE_OUT)) {  // the dense gate from the tiled gate epilogue
    if (srw::tiled_supports(d)) return 2;
    if (srw::tiled_f32_supports(d)) return 3;
  } else if (!force_generic) {
    if ((d.flags & SRW_FLAG_TILED) && srw::tiled_supports(d)) return 2;
    if (srw::mfma_supports(d, h_is_x)) return 1;
    if (srw::tiled_supports(d)) return 2;
    if (srw::tiled_f32_supports(d)) return 3;
  }
  if (d.stats_mode == SRW_STATS_GRAM) return -1;  // only the MFMA family implements it
  if (srw::generic_supports(d)) return 0;  // dense under SRW_FLAG_SPARSE_SKIP
  return -1;
}

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Device address of `scratch` per device, looked up once per device, with
// that device current, on the first no-allocation call that runs there.
// That call may come while the caller's stream is being captured into a HIP
// graph: the lookup (no stream work) runs with this thread's capture mode
// relaxed, so that a capture in global mode does not refuse it.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

srw_status_t scratch_address(hipStream_t stream, void** out) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return SRW_EHIP;
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd;
    if (hipStreamGetDevice(stream, &sd) != hipSuccess) return SRW_EHIP;
    dev = static_cast<int>(sd);
  }
  if (dev < 0 || dev >= kMaxDevices) return SRW_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return SRW_EHIP;
    hipError_t e = hipSuccess;
    if (dev != cur) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    (void)hipThreadExchangeStreamCaptureMode(&mode);  // the caller's mode back
    if (e != hipSuccess || p == nullptr) return SRW_EHIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SRW_OK;
}

size_t bytes_of(int which, const srw_desc_t& d) {
  if (which == 1) return srw::mfma_workspace_bytes(d);
  if (which == 2) return srw::tiled_workspace_bytes(d);
  if (which == 3) return srw::tiled_f32_workspace_bytes(d);
  return srw::generic_workspace_bytes(d);
}

}  // namespace

namespace srw {
void dominant_kernel_begin(hipStream_t s) {
  if (g_ev_start && g_ev_stop) (void)hipEventRecord(g_ev_start, s);
}
void dominant_kernel_end(hipStream_t s) {
  if (g_ev_start && g_ev_stop) (void)hipEventRecord(g_ev_stop, s);
}
}  // namespace srw

extern "C" {

int32_t srw_abi_version(void) { return SRW_AMD_ABI_VERSION; }

const char* srw_status_string(srw_status_t s) {
  // A C caller may pass any int here; read its bits as an int (loading a C++
  // enum outside its enumerators' range is undefined behaviour)
  static_assert(sizeof(srw_status_t) == sizeof(int32_t), "srw_status_t is int-sized");
  int32_t v;
  memcpy(&v, &s, sizeof v);
  switch (v) {
    case SRW_OK: return "SRW_OK";
    case SRW_EINVAL: return "SRW_EINVAL: invalid argument";
    case SRW_EUNSUPPORTED: return "SRW_EUNSUPPORTED: configuration not implemented";
    case SRW_EHIP: return "SRW_EHIP: HIP runtime error";
    case SRW_EWORKSPACE: return "SRW_EWORKSPACE: workspace missing or too small";
    case SRW_ESCRATCH:
      return "SRW_ESCRATCH: the call needs more workspace than srw_forward_noalloc's scratch holds "
             "(SRW_NOALLOC_SCRATCH_BYTES = 64 MiB); use srw_forward with a workspace";
  }
  return "SRW_?: unknown status";
}

srw_status_t srw_desc_init(srw_desc_t* d) {
  if (!d) return SRW_EINVAL;
  memset(d, 0, sizeof(*d));
  d->n_routes = 1;
  d->dtype = SRW_BF16;
  d->gate = SRW_GATE_V41;
  d->stats_mode = SRW_STATS_ONEPASS;
  d->sharpness = 500.0f;       // v41:297
  d->act_threshold = 0.5f;     // v41:298
  d->act_cutoff = 0.01f;       // v41:299
  d->epsilon = 1e-4f;          // v41:300
  d->max_intensity = 10.0f;    // v41:301
  d->dead_threshold = 0.01f;   // v41:352
  d->scale = 1.0f;
  d->chunk_size = 0;
  d->flags = 0;
  return SRW_OK;
}

srw_status_t srw_workspace_size(const srw_desc_t* d, size_t* bytes) {
  srw_status_t st = validate(d);
  if (st != SRW_OK) return st;
  if (!bytes) return SRW_EINVAL;
  // the largest need over the paths a call may take: h aliasing x (possible
  // when d_route == d_model with one route) can select the MFMA family
  const bool can_alias = d->n_routes == 1 && d->d_route == d->d_model;
  const int which = choose(*d, false);
  const int which_alias = can_alias ? choose(*d, true) : which;
  if (which < 0 && which_alias < 0) return SRW_EUNSUPPORTED;
  size_t need = 0;
  for (int w : {which, which_alias}) {
    if (w < 0 || d->T == 0) continue;  // no tokens: srw_forward needs no workspace
    const size_t n = align256(bytes_of(w, *d));
    need = n > need ? n : need;
  }
  *bytes = need;
  return SRW_OK;
}

}  // extern "C"

namespace {
// Validation and launch arguments of one srw_forward call; *which = the kernel
// family (or -2: no tokens, nothing to launch).
srw_status_t prepare_forward(const srw_desc_t* d, const srw_tensors_t* in, const srw_outputs_t* o, void* workspace,
                             size_t workspace_bytes, void* stream, srw::LaunchArgs* a, int* which) {
  srw_status_t st = validate(d);
  if (st != SRW_OK) return st;
  if (!in || !o) return SRW_EINVAL;
  int w = choose(*d, in->h != nullptr && in->h == in->x);
  // the dense gate: the tiled families under SRW_FLAG_GATE_OUT, else the generic kernels
  if (w > 0 && o->gate && !((d->flags & SRW_FLAG_GATE_OUT) && (w == 2 || w == 3)))
    w = srw::generic_supports(*d) ? 0 : -1;
  if (w < 0) return SRW_EUNSUPPORTED;
  if (d->T == 0) {  // nothing to compute; empty tensors may carry null pointers
    *which = -2;
    return SRW_OK;
  }
  if (!in->x || !in->h || !in->emb || !in->tau_offset || !in->read || !in->write || !o->out) return SRW_EINVAL;
  if (in->h == in->x && !(d->n_routes == 1 && d->d_route == d->d_model)) return SRW_EINVAL;
  const size_t need = align256(bytes_of(w, *d));
  if (need > 0 && (!workspace || workspace_bytes < need)) return SRW_EWORKSPACE;

  *a = srw::LaunchArgs{};
  a->d = *d;
  a->in = *in;
  a->o = *o;
  if (!(d->flags & SRW_FLAG_DIAG)) {
    a->o.token_diag = nullptr;
    a->o.unit_diag = nullptr;
  }
  a->gp.sharp = d->sharpness;
  a->gp.thr = d->act_threshold;
  a->gp.cut = d->act_cutoff;
  a->gp.eps = d->epsilon;
  a->gp.maxi = d->max_intensity;
  a->gp.cap_thresh = (d->epsilon + d->max_intensity) - 1e-3f;  // v41:487 in float32
  a->words = (d->n_units + 63) / 64;
  a->chunk = (d->chunk_size > 0 && d->chunk_size < d->n_units) ? d->chunk_size : d->n_units;
  a->ws = static_cast<char*>(workspace);
  a->ws_bytes = workspace_bytes;
  a->stream = static_cast<hipStream_t>(stream);
  *which = w;
  return SRW_OK;
}

srw_status_t launch_forward(const srw::LaunchArgs& a, int which) {
  (void)hipGetLastError();  // start from a clean error state
  hipError_t e;
  if (which == 1) {
    const char* name = "mfma";
    e = srw::mfma_forward(a, &name);
    g_last_path = name;
  } else if (which == 2) {
    e = srw::tiled_forward(a);
    g_last_path = srw::tiled_runs_sparse(a.d) ? "tiled_sparse_bf16" : "tiled_bf16";
  } else if (which == 3) {
    e = srw::tiled_f32_forward(a);
    g_last_path = "tiled_f32";
  } else {
    e = srw::generic_forward(a);
    g_last_path = "generic";
  }
  return e == hipSuccess ? SRW_OK : SRW_EHIP;
}
}  // namespace

extern "C" {

srw_status_t srw_forward(const srw_desc_t* d, const srw_tensors_t* in, const srw_outputs_t* o, void* workspace,
                         size_t workspace_bytes, void* stream) {
  srw::LaunchArgs a;
  int which = -1;
  const srw_status_t st = prepare_forward(d, in, o, workspace, workspace_bytes, stream, &a, &which);
  if (st != SRW_OK) return st;
  if (which == -2) {
    g_last_path = "empty";
    return SRW_OK;
  }
  return launch_forward(a, which);
}

srw_status_t srw_forward_noalloc(const srw_desc_t* d, const srw_tensors_t* in, const srw_outputs_t* o,
                                 void* stream) {
  srw_status_t st = validate(d);
  if (st != SRW_OK) return st;
  // the scratch keeps whatever the last call on this GPU left there: a pool
  // packed by another call must not be taken for this call's
  if (d->flags & SRW_FLAG_POOL_CACHED) return SRW_EINVAL;
  size_t need = 0;
  if ((st = srw_workspace_size(d, &need)) != SRW_OK) return st;
  if (need > SRW_NOALLOC_SCRATCH_BYTES) return SRW_ESCRATCH;
  void* ws = nullptr;
  if (need > 0 && (st = scratch_address(static_cast<hipStream_t>(stream), &ws)) != SRW_OK) return st;
  return srw_forward(d, in, o, ws, need > 0 ? SRW_NOALLOC_SCRATCH_BYTES : 0, stream);
}

srw_status_t srw_workspace_size_batch(int32_t n, const srw_desc_t* descs, size_t* bytes) {
  if (n < 1 || n > SRW_MAX_BATCH || !descs || !bytes) return SRW_EINVAL;
  size_t total = 0;
  for (int32_t i = 0; i < n; ++i) {
    size_t b = 0;
    const srw_status_t st = srw_workspace_size(&descs[i], &b);
    if (st != SRW_OK) return st;
    total += align256(b);
  }
  *bytes = total;
  return SRW_OK;
}

srw_status_t srw_forward_batch(int32_t n, const srw_desc_t* descs, const srw_tensors_t* ins,
                               const srw_outputs_t* outs, void* workspace, size_t workspace_bytes, void* stream) {
  if (n < 1 || n > SRW_MAX_BATCH || !descs || !ins || !outs) return SRW_EINVAL;
  size_t need = 0;
  srw_status_t st = srw_workspace_size_batch(n, descs, &need);
  if (st != SRW_OK) return st;
  if (need > 0 && (!workspace || workspace_bytes < need)) return SRW_EWORKSPACE;
  // call i's workspace slice: the aligned sizes of calls 0 .. i-1 before it
  srw::LaunchArgs a[SRW_MAX_BATCH];
  int which[SRW_MAX_BATCH];
  size_t off = 0;
  bool all_mfma = true;
  for (int32_t i = 0; i < n; ++i) {
    size_t b = 0;
    (void)srw_workspace_size(&descs[i], &b);
    b = align256(b);
    char* ws = b > 0 ? static_cast<char*>(workspace) + off : nullptr;
    st = prepare_forward(&descs[i], &ins[i], &outs[i], ws, b, stream, &a[i], &which[i]);
    if (st != SRW_OK) return st;
    all_mfma = all_mfma && which[i] == 1;
    off += b;
  }
  if (all_mfma && n > 1) {
    (void)hipGetLastError();
    const char* name = "mfma";
    const hipError_t e = srw::mfma_forward_batch(a, n, &name);
    if (e == hipSuccess) {
      g_last_path = name;
      return SRW_OK;
    }
    if (e != hipErrorNotSupported) return SRW_EHIP;
  }
  for (int32_t i = 0; i < n; ++i) {  // one after the other
    if (which[i] == -2) continue;
    st = launch_forward(a[i], which[i]);
    if (st != SRW_OK) return st;
  }
  if (n > 1) g_last_path = "batch_sequential";
  return SRW_OK;
}

srw_status_t srw_backward_workspace_size(const srw_desc_t* d, size_t* bytes) {
  srw_status_t st = validate(d);
  if (st != SRW_OK) return st;
  if (!bytes) return SRW_EINVAL;
  if (!srw::tiled_backward_supports(*d)) return SRW_EUNSUPPORTED;
  *bytes = d->T == 0 ? 0 : align256(srw::tiled_backward_workspace_bytes(*d));
  return SRW_OK;
}

srw_status_t srw_backward(const srw_desc_t* d, const srw_tensors_t* in, const srw_cotangents_t* cot,
                          const srw_grads_t* grads, void* workspace, size_t workspace_bytes, void* stream) {
  srw_status_t st = validate(d);
  if (st != SRW_OK) return st;
  if (!in || !cot || !grads) return SRW_EINVAL;
  if (!srw::tiled_backward_supports(*d)) return SRW_EUNSUPPORTED;
  if (d->T == 0) {  // no tokens: the pool gradients are zero
    if (!grads->demb || !grads->dread || !grads->dwrite) return SRW_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t N = d->n_units;
    if (srw::fill_f32(grads->demb, N * d->d_route, 0.f, s) != hipSuccess ||
        srw::fill_f32(grads->dread, N * d->d_model, 0.f, s) != hipSuccess ||
        srw::fill_f32(grads->dwrite, N * d->d_model, 0.f, s) != hipSuccess ||
        (grads->dscale && srw::fill_f32(grads->dscale, 1, 0.f, s) != hipSuccess))
      return SRW_EHIP;
    g_last_path = "empty";
    return SRW_OK;
  }
  if (!in->x || !in->h || !in->emb || !in->tau_offset || !in->read || !in->write) return SRW_EINVAL;
  if (!cot->d_out || !cot->out) return SRW_EINVAL;
  if (!cot->den != !cot->unit_diag) return SRW_EINVAL;  // the forward's residuals: both or neither
  if (!grads->dx || !grads->dh || !grads->demb || !grads->dtau_offset || !grads->dread || !grads->dwrite)
    return SRW_EINVAL;
  // rows are read and written in 16-byte pieces
  for (const void* p : {in->x, in->h, in->emb, in->read, in->write, cot->out, static_cast<const void*>(cot->d_out),
                        static_cast<const void*>(grads->dx), static_cast<const void*>(grads->dh),
                        static_cast<const void*>(grads->demb), static_cast<const void*>(grads->dread),
                        static_cast<const void*>(grads->dwrite)})
    if (reinterpret_cast<uintptr_t>(p) & 15) return SRW_EINVAL;
  if (!isfinite(cot->d_score_lb) || !isfinite(cot->d_dead_penalty)) return SRW_EINVAL;
  // the v4.0.1 fused function has no dead-unit penalty (v401:343-367)
  if (d->gate == SRW_GATE_GELU_V401 && cot->d_dead_penalty != 0.0f) return SRW_EINVAL;
  const size_t need = align256(srw::tiled_backward_workspace_bytes(*d));
  if (!workspace || workspace_bytes < need) return SRW_EWORKSPACE;
  srw::BackwardArgs a{};
  a.d = *d;
  a.in = *in;
  a.cot = *cot;
  a.g = *grads;
  a.gp.sharp = d->sharpness;
  a.gp.thr = d->act_threshold;
  a.gp.cut = d->act_cutoff;
  a.gp.eps = d->epsilon;
  a.gp.maxi = d->max_intensity;
  a.gp.cap_thresh = (d->epsilon + d->max_intensity) - 1e-3f;
  a.ws = static_cast<char*>(workspace);
  a.ws_bytes = workspace_bytes;
  a.stream = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const hipError_t e = srw::tiled_backward(a);
  g_last_path = "tiled_bwd_bf16";
  return e == hipSuccess ? SRW_OK : SRW_EHIP;
}

const char* srw_last_path(void) { return g_last_path; }

srw_status_t srw_set_kernel_events(void* start, void* stop) {
  if ((start == nullptr) != (stop == nullptr)) return SRW_EINVAL;
  g_ev_start = static_cast<hipEvent_t>(start);
  g_ev_stop = static_cast<hipEvent_t>(stop);
  return SRW_OK;
}

}  // extern "C"

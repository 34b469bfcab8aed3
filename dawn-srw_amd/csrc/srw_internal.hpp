// srw_internal.hpp -- host-side launch interface between the C ABI layer
// (srw_capi.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srw_amd.h"
#include "srw_common.hpp"

namespace srw {

// Everything a kernel family needs for one srw_forward call, with pointers
// already offset and validated by the ABI layer.
struct LaunchArgs {
  srw_desc_t d;
  srw_tensors_t in;
  srw_outputs_t o;
  GateParams gp;
  int64_t words;     // ceil(N / 64): pass_mask words per (token, route)
  int64_t chunk;     // N-chunk size of the reference plan (emulation); N if none
  char* ws;          // workspace base (may be null when none is needed)
  size_t ws_bytes;
  hipStream_t stream;
};

// Generic kernels: one workgroup per (token, route), scalar FMA, faithful
// to every reference rounding point.  Any shape with D <= 4096.
size_t generic_workspace_bytes(const srw_desc_t& d);
bool generic_supports(const srw_desc_t& d);
hipError_t generic_forward(const LaunchArgs& a);

// Profiling hook (srw_set_kernel_events): brackets the dominant kernel of a
// call with the caller's events, when the calling thread installed them.
void dominant_kernel_begin(hipStream_t s);
void dominant_kernel_end(hipStream_t s);

// Fill kernel (graph-safe replacement for hipMemsetAsync).
hipError_t fill_f32(float* p, int64_t n, float v, hipStream_t s);

// dst row n = src row n / (||src row n|| + 1e-8) in bf16 for N rows of D
// (v4.0.1 forward normalisation of the read / write rows, v401:300-301),
// see srw_generic.hip.
hipError_t normalize_rows_bf16(const uint16_t* src, uint16_t* dst, int64_t N, int64_t D, hipStream_t s);
// r / (||r|| + 1e-8) per row in fp32 (v401:1456-1457), one workgroup per row
hipError_t normalize_rows_f32(const float* src, float* dst, int64_t N, int64_t D, hipStream_t s);

// Pack a bf16 [N, D] matrix unit-contiguous in matrix-core fragment order
// (32-unit tiles; tail units zero), see srw_mfma.hip.
hipError_t pack_unit_major(const uint16_t* src, uint16_t* dst, int64_t N, int D, hipStream_t s);

// out[r][u] = bf16(a[r] . b[u]) for r < rows and u < ceil(n / 32) * 32 (b's
// rows past n repeat its last row), row stride ld elements, with a [rows, k]
// and b [n, k] bf16 row-major, on the moments kernel's tile loop
// (srw_mfma.hip).  With mom non-null also the per-split moment partials
// mom[rows_gemm_splits(rows, n)][rows][2] = (sum, sum of squares) of each
// row's bf16 values over the units [0, n).  k: 32, 64, 128 or 384.
bool rows_gemm_supports(int64_t k);
int rows_gemm_splits(int64_t rows, int64_t n);
hipError_t rows_gemm(const uint16_t* a, int64_t rows, const uint16_t* b, int64_t n, int64_t k, uint16_t* out,
                     int64_t ld, float* mom, hipStream_t s);

// Gram statistics (SRW_STATS_GRAM), see srw_gram.hip: writes the per-token
// moment partials mom[gram_moment_parts(dr)][T][2] = (sum s, sum s^2).
bool gram_supports(int64_t dr);
int gram_moment_parts(int64_t dr);
size_t gram_workspace_bytes(int64_t N, int64_t dr);
// Also zeroes the pass-mask words that two N-splits share (chunk boundaries
// inside a 32-unit tile of chunk size cs) and the unused half of the last word.
// pool_cached: G and esum of this pool are already in `ws` from an earlier call.
hipError_t gram_moments(const uint16_t* emb, const uint16_t* h, int64_t T, int64_t N, int64_t dr, float* mom,
                        char* ws, hipStream_t s, uint32_t* mask32, int64_t words32, int64_t cs, int nc,
                        bool pool_cached);

// Per-row tau from moment partials mom[S_st][T][ms] (srw_mfma.hip).
// kTauOnePass: std = sqrt(E[s^2] - mean^2) + 1e-8 (v41:461-462);
// kTauChan: the centred std = sqrt(sum (s - mean)^2 / N) + 1e-8
// (v41:1719-1721) from per-partial (sum s, sum (s - partial mean)^2)
// over upp consecutive units each (partial i: units [upp i, upp i + upp) of
// the N; upp = 0: the partial's count in its third float, ms = 3), merged
// by Chan et al.'s parallel formula M2 = sum M2_i + sum n_i (mean_i -
// mean)^2 -- the centred sum of squares without a second pass over the
// scores.
enum TauMode { kTauOnePass = 0, kTauChan = 3 };
// sstd (or null): the row's s_std as well (the v4.0.1 gate's z scale).
hipError_t launch_tau(const float* mom, const float* tau_off, float* tau, int64_t T, int S_st, int64_t N, int ms,
                      float* token_diag, int mode, hipStream_t s, float* sstd = nullptr, int upp = 0);

// Final reduction over N-splits (srw_mfma.hip): sums the fp32 partial outputs
// out_part[S][T][D] split by split, rounds each reference chunk (spc
// consecutive splits) to bf16, den = max(sum intensity, 1) (v4.1, v41:584)
// or max(sum gate, 1) (den_gate: the v4.0.1 gate, v401:340) from
// tok_part[S_tok][T][tps] = (sum gate, sum intensity or z+, active count,
// ...), out = bf16(bf16(raw / den) * scale).
struct FinalizeArgs {
  const float* out_part;
  const float* tok_part;
  uint16_t* out;
  float* gate_sum;
  float* den;
  int32_t* n_active;
  int64_t T;
  int D, S, spc, S_tok, tps;
  float scale;
  const float* tau;    // diagnostics only
  float* token_diag;   // [T][SRW_TDIAG_COUNT] or null
  GateParams gp;
  float exp_scale;
  int den_gate;        // den from the gate sum (v4.0.1)
};
hipError_t launch_finalize(const FinalizeArgs& f, hipStream_t s);

// Everything the backward needs for one srw_backward call.
struct BackwardArgs {
  srw_desc_t d;
  srw_tensors_t in;
  srw_cotangents_t cot;
  srw_grads_t g;
  GateParams gp;
  char* ws;
  size_t ws_bytes;
  hipStream_t stream;
};

// Backward (VJP) on the tiled MFMA kernels, see srw_tiled.hip.
bool tiled_backward_supports(const srw_desc_t& d);
size_t tiled_backward_workspace_bytes(const srw_desc_t& d);
hipError_t tiled_backward(const BackwardArgs& a);

// Tiled-GEMM kernels for wide layers (bf16), see srw_tiled.hip: P = gated
// product materialised in HBM; d_model and d_route multiples of 64.
bool tiled_supports(const srw_desc_t& d);
size_t tiled_workspace_bytes(const srw_desc_t& d);
bool tiled_runs_sparse(const srw_desc_t& d);  // SRW_FLAG_SPARSE_SKIP at a width the sparse kernels take
hipError_t tiled_forward(const LaunchArgs& a);

// fp32 tiled GEMMs on the fp32 matrix cores, see srw_tiled_f32.hip: the v4.1
// gate with one-pass or centred statistics (the fp32 _srw_inference);
// d_model and d_route multiples of 32.
bool tiled_f32_supports(const srw_desc_t& d);
size_t tiled_f32_workspace_bytes(const srw_desc_t& d);
hipError_t tiled_f32_forward(const LaunchArgs& a);

// MFMA kernels (bf16 / f32 matrix cores), see srw_mfma.hip.
size_t mfma_workspace_bytes(const srw_desc_t& d);
// h_is_x: h aliases x (d_route == d_model, one route), which some shapes need
bool mfma_supports(const srw_desc_t& d, bool h_is_x);
hipError_t mfma_forward(const LaunchArgs& a, const char** path_name);
// Up to four decode-shaped calls in one launch per stage (srw_forward_batch);
// hipErrorNotSupported, with nothing launched, when they cannot share one.
hipError_t mfma_forward_batch(const LaunchArgs* a, int n, const char** path_name);

}  // namespace srw

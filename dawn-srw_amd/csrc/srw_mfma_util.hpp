// srw_mfma_util.hpp -- gfx950 matrix-core and LDS helpers shared by the
// bf16 kernel families (srw_mfma.hip, srw_gemm.hip).
//
// v_mfma_f32_32x32x16_bf16 operand layout (wave64):
//   A operand: lane l holds A[l % 32][8 (l / 32) + i], i = 0..7
//   B operand: lane l holds B[8 (l / 32) + i][l % 32]
//   C/D:       acc[v] of lane l is C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32]
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace srw {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kFragBytes = 1024;  // one MFMA operand fragment: 64 lanes x 16 B

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ inline f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Two floats -> two bf16 (round to nearest even, v_cvt_pk_bf16_f32), low = first.
__device__ inline uint32_t pack_bf16(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ inline float lo_f32(uint32_t p) { return __uint_as_float(p << 16); }
__device__ inline float hi_f32(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// Unit (within a 32-unit tile) carried by k index 8*half + i of k-step j of
// the write GEMM: the accumulator row of score-GEMM register v = 8 j + i.
// (A 32 x 32 accumulator -- rows = units, lane = token -- is the A operand of
// the write GEMM under this unit permutation.)
__host__ __device__ inline int unit_of_k(int j, int half, int i) {
  return 16 * j + 8 * (i >> 2) + 4 * half + (i & 3);
}
// Unit (within the tile) of score-accumulator register v in lane-half `half`.
__device__ inline int unit_of_acc(int v, int half) { return 8 * (v >> 2) + 4 * half + (v & 3); }

// One 16-byte direct global->LDS load per lane; the LDS destination of the
// wave is `lds` (wave-uniform) + 16 * lane.
__device__ inline void g2lds16(const void* g, char* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 16, 0, 0);
}
// The same with the non-temporal (streaming) cache policy, for data read
// once: it does not displace data other workgroups or kernels reuse.
__device__ inline void g2lds16_nt(const void* g, char* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 16, 0, 2);  // cache policy bit 1: nt
}

__device__ inline void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Workgroup barrier that waits only for this wave's LDS operations.
// __syncthreads() is a workgroup-scope release/acquire, for which the
// compiler also drains every global load in flight (vmcnt(0)) -- including
// the global->LDS prefetch of later tiles.  Here global->LDS loads stay in
// flight; a caller that publishes them waits for them first.  The
// compiler-only fences keep memory accesses on their side of the barrier.
__device__ inline void barrier_lds() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// v4.0.1 GELU gate of a score s (v401:303-306): z = (s - tau) / s_std,
// Phi(z) = 0.5 (1 + erf(z / sqrt 2)), gate = z Phi(z) for z > 0, else 0.
// zpos = max(z, 0) (the row's z sum, v401:314); the unit passes <=> z > 0
// <=> s > tau, the sign bit of tau - s.  inv_std = 1 / s_std of the row.
// raw_bf16: s - tau rounded to bf16, as _srw_inference computes it in the
// scores' dtype (v401:1451-1452; tau is then bf16 as well).
// erf of the non-negative argument by Abramowitz & Stegun 7.1.26:
// erf(x) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^(-x^2),
// t = 1 / (1 + p x), |error| <= 1.5e-7 -- a few registers, where the
// library erff spills the kernels' registers.
__device__ inline float gelu_gate(float s, float tau, float inv_std, float& zpos, bool raw_bf16 = false) {
  float raw = s - tau;
  if (raw_bf16) raw = __uint_as_float(pack_bf16(0.0f, raw));  // the high half: bf16(raw)
  const float z = raw * inv_std;
  const float x = fmaxf(z, 0.0f) * 0.7071067811865476f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, x, 1.0f));
  float q = fmaf(1.061405429f, t, -1.453152027f);
  q = fmaf(q, t, 1.421413741f);
  q = fmaf(q, t, -0.284496736f);
  q = fmaf(q, t, 0.254829592f);
  const float erf = 1.0f - q * t * __builtin_amdgcn_exp2f(-x * x * 1.4426950408889634f);
  zpos = z > 0.0f ? z : 0.0f;
  return z > 0.0f ? z * (0.5f * (1.0f + erf)) : 0.0f;
}

}  // namespace srw

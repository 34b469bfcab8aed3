// srw_common.hpp -- device helpers shared by the SRW kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "srw_amd.h"

namespace srw {

constexpr int kWave = 64;

// bf16 storage type: raw bits, converted with explicit round-to-nearest-even
// so that every rounding point is under our control (the reference rounds
// dot outputs, gates and products to bf16, v41:439, 503, 516-518).
struct bf16_t {
  uint16_t bits;
};

__host__ __device__ inline float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__host__ __device__ inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_bits(f)); }

template <typename T> struct Elt;
template <> struct Elt<float> {
  static __device__ inline float load(const float* p) { return *p; }
  static __device__ inline void store(float* p, float v) { *p = v; }
  // rounding of a dot product / elementwise result to the storage dtype
  static __device__ inline float round(float v) { return v; }
};
template <> struct Elt<bf16_t> {
  static __device__ inline float load(const bf16_t* p) { return bf16_to_f32(p->bits); }
  static __device__ inline void store(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); }
  static __device__ inline float round(float v) { return round_bf16(v); }
};

// Gate constants as float32, exactly as the reference closure bakes them
// (jnp.float32(...) at v41:379-383).
struct GateParams {
  float sharp, thr, cut, eps, maxi;
  float cap_thresh;  // eps + maxi - 1e-3 (v41:487), computed in float32
};

struct GateOut {
  float margin, act, inten, gate;
};

// v4.1 two-stage gate, v41:506-511 (same expression order, float32).
__device__ inline GateOut gate_v41(float s, float tau, const GateParams& g) {
  GateOut o;
  float raw = s - tau;
  o.margin = raw - g.thr;
  o.act = 1.0f / (1.0f + expf(-(g.sharp * o.margin)));
  float am = fmaxf(o.margin - g.cut, 0.0f);
  o.inten = g.eps + fminf(am, g.maxi);
  o.gate = o.act * o.inten;
  return o;
}

// v4.0.1 GELU gate, v401:305-310: z = raw/std, gate = z Phi(z) for z > 0.
struct GeluOut {
  float z, phi, gate;
};
__device__ inline GeluOut gate_gelu_v401(float s, float tau, float s_std) {
  GeluOut o;
  float raw = s - tau;
  o.z = raw / s_std;
  o.phi = 0.5f * (1.0f + erff(o.z * 0.7071067811865476f));
  o.gate = o.z > 0.0f ? o.z * o.phi : 0.0f;
  return o;
}

// ---- wave / block reductions (fixed order => deterministic) --------------

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Sum of `v` over a block of NT threads; every thread gets the result.
// `red` must hold NT/64 floats of LDS.
template <int NT>
__device__ inline float block_sum(float v, float* red) {
  constexpr int NW = NT / kWave;
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) r += red[i];
  return r;
}
template <int NT>
__device__ inline float block_max(float v, float* red) {
  constexpr int NW = NT / kWave;
  v = wave_max(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, red[i]);
  return r;
}

// atomic max for non-negative floats (their bit patterns order like uints)
__device__ inline void atomic_max_nonneg(float* addr, float v) {
  if (!(v >= 0.0f)) return;
  atomicMax(reinterpret_cast<unsigned int*>(addr), __float_as_uint(v));
}

}  // namespace srw

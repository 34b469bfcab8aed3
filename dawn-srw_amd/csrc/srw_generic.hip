// srw_generic.hip -- generic SRW forward: one workgroup per (token, route).
//
// This family follows the reference's arithmetic step by step (scores rounded
// to the storage dtype, v41:439/503; gate rounded to bf16, v41:516; x.R^T
// rounded, v41:517; gate*xr rounded, v41:518; optionally the per-chunk bf16
// rounding of the write GEMM output, v41:518 with the chunk plan of
// v41:416-420; out/den rounded to bf16, v41:586).  It handles every shape
// (ragged N, any d_model <= 4096, any d_route) and both gates, and is the
// reference-faithful path the MFMA kernels are tested against on the GPU.
//
// Work per workgroup: sweep 1 computes the token's score moments over all N
// (two sweeps for the centred variance), sweep 2 recomputes each score,
// gates it, computes x.r_n, stages gate*xr in LDS and accumulates
// sum_n p_n w_n[d] with one thread per output column d.

#include "srw_internal.hpp"

namespace srw {

namespace {

constexpr int kGT = 256;       // threads per workgroup
constexpr int kGMaxDPT = 16;   // output columns per thread -> d_model <= 4096

struct GenericParams {
  const void* x;
  const void* h;
  const void* emb;
  const float* tau_off;
  const void* read;    // read rows (forward-normalised copy for v4.0.1)
  const void* write;   // write rows (forward-normalised copy for v4.0.1)
  void* out;
  float* gate_sum;
  float* den;
  int32_t* n_active;
  uint64_t* pass_mask;
  float* token_diag;
  float* unit_diag;
  float* gate_out;     // [T, R, N] or null
  int64_t D, dr, N, words, chunk;
  int R;
  int stats;
  GateParams gp;
  float scale;
};

template <typename E>
__device__ inline float dot_row(const float* __restrict__ v, const E* __restrict__ row, int64_t K) {
  float acc = 0.0f;
  for (int64_t k = 0; k < K; ++k) acc = fmaf(v[k], Elt<E>::load(row + k), acc);
  return acc;
}

template <typename E, bool V401, bool EMU, bool DIAG>
__global__ __launch_bounds__(kGT) void srw_generic_kernel(GenericParams a) {
  const int64_t tr = blockIdx.x;  // token * R + route
  const int64_t t = tr / a.R;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  extern __shared__ float smem[];
  float* hs = smem;          // [dr]
  float* xs = hs + a.dr;     // [D]
  float* ps = xs + a.D;      // [kGT]
  float* red = ps + kGT;     // [kGT / 64]

  const E* X = static_cast<const E*>(a.x) + t * a.D;
  const E* H = static_cast<const E*>(a.h) + tr * a.dr;
  for (int64_t i = tid; i < a.dr; i += kGT) hs[i] = Elt<E>::load(H + i);
  for (int64_t i = tid; i < a.D; i += kGT) xs[i] = Elt<E>::load(X + i);
  __syncthreads();

  const E* Em = static_cast<const E*>(a.emb);
  const E* Rm = static_cast<const E*>(a.read);
  const E* Wm = static_cast<const E*>(a.write);
  const int64_t N = a.N;
  const float fN = static_cast<float>(N);

  // ---- sweep 1: score moments (v41:434-462 one-pass; v41:1719-1721 centred)
  float s_mean, s_std, m3 = 0.0f, m4 = 0.0f;
  if (a.stats == SRW_STATS_ONEPASS) {
    float s1 = 0.f, s2 = 0.f, s3 = 0.f, s4 = 0.f;
    for (int64_t n = tid; n < N; n += kGT) {
      const float s = Elt<E>::round(dot_row(hs, Em + n * a.dr, a.dr));
      const float sq = s * s;
      s1 += s;
      s2 += sq;
      s3 += sq * s;
      s4 += sq * sq;
      if (DIAG && a.unit_diag) atomicAdd(a.unit_diag + n * SRW_UDIAG_COUNT + SRW_UDIAG_SCORE_SUM, s);
    }
    const float S1 = block_sum<kGT>(s1, red);
    const float S2 = block_sum<kGT>(s2, red);
    s_mean = S1 / fN;
    s_std = sqrtf(S2 / fN - s_mean * s_mean) + 1e-8f;
    if (DIAG) {
      m3 = block_sum<kGT>(s3, red);
      m4 = block_sum<kGT>(s4, red);
    }
  } else {
    float s1 = 0.f;
    for (int64_t n = tid; n < N; n += kGT) {
      const float s = Elt<E>::round(dot_row(hs, Em + n * a.dr, a.dr));
      s1 += s;
      if (DIAG && a.unit_diag) atomicAdd(a.unit_diag + n * SRW_UDIAG_COUNT + SRW_UDIAG_SCORE_SUM, s);
    }
    s_mean = block_sum<kGT>(s1, red) / fN;
    float s2 = 0.f;
    for (int64_t n = tid; n < N; n += kGT) {
      const float s = Elt<E>::round(dot_row(hs, Em + n * a.dr, a.dr));
      const float dv = s - s_mean;
      s2 += dv * dv;
    }
    s_std = sqrtf(block_sum<kGT>(s2, red) / fN) + 1e-8f;
  }
  const float tau = s_mean + a.tau_off[tr] * s_std;

  // ---- sweep 2: gate, read, gated write (v41:503-534)
  const int nd = static_cast<int>((a.D + kGT - 1) / kGT);
  float acc[kGMaxDPT], tot[kGMaxDPT];
#pragma unroll
  for (int j = 0; j < kGMaxDPT; ++j) {
    acc[j] = 0.f;
    tot[j] = 0.f;
  }
  float gsum = 0.f, isum = 0.f, nact = 0.f;
  float gmax = -1e9f, nstrong = 0.f, nbound = 0.f, n075 = 0.f, n030 = 0.f;
  float glogg = 0.f, imax = 0.f, ncap = 0.f;
  int64_t chunk_end = a.chunk;
  uint64_t* mask_row = a.pass_mask ? a.pass_mask + tr * a.words : nullptr;

  for (int64_t base = 0; base < N; base += kGT) {
    const int64_t n = base + tid;
    float p = 0.f;
    bool active = false;
    if (n < N) {
      const float s = Elt<E>::round(dot_row(hs, Em + n * a.dr, a.dr));
      float gate;
      if (!V401) {
        const GateOut g = gate_v41(s, tau, a.gp);
        gate = g.gate;
        active = g.act > 0.5f;
        isum += g.inten;
        if (DIAG) {
          nstrong += g.act > 0.9f ? 1.f : 0.f;
          nbound += (g.act > 0.1f && g.act < 0.9f) ? 1.f : 0.f;
          n075 += (g.act > 0.05f && g.act < 0.95f) ? 1.f : 0.f;
          n030 += (g.act > 0.2f && g.act < 0.8f) ? 1.f : 0.f;
          imax = fmaxf(imax, g.inten);
          ncap += g.inten >= a.gp.cap_thresh ? 1.f : 0.f;
        }
      } else {
        const GeluOut g = gate_gelu_v401(s, tau, s_std);
        gate = g.gate;
        active = g.gate > 0.0f;                 // v401:316
        isum += g.z > 0.f ? g.z : 0.f;          // v401:319 (z_sum)
        if (DIAG) {
          nstrong += g.gate > 0.5f ? 1.f : 0.f;
          nbound += (g.phi > 0.95f || g.phi < 0.05f) ? 1.f : 0.f;
          n075 += (g.z > 0.f && g.z < 0.75f) ? 1.f : 0.f;
          n030 += (g.z > 0.f && g.z < 0.30f) ? 1.f : 0.f;
        }
      }
      gsum += gate;
      nact += active ? 1.f : 0.f;
      if (a.gate_out) a.gate_out[tr * N + n] = gate;   // gate_raw (v41:1760, 1769)
      if (DIAG) {
        gmax = fmaxf(gmax, gate);
        glogg += gate * logf(gate + 1e-8f);
        if (a.unit_diag) atomic_max_nonneg(a.unit_diag + n * SRW_UDIAG_COUNT + SRW_UDIAG_GATE_MAX, gate);
      }
      const float xr = Elt<E>::round(dot_row(xs, Rm + n * a.D, a.D));
      p = Elt<E>::round(Elt<E>::round(gate) * xr);
    }
    const uint64_t m = __ballot(active);
    if (mask_row && lane == 0 && base + kWave * wave < N) mask_row[base / kWave + wave] = m;
    ps[tid] = p;
    __syncthreads();
    const int cnt = static_cast<int>(N - base < kGT ? N - base : kGT);
    for (int j = 0; j < cnt; ++j) {
      if (EMU && base + j == chunk_end) {
#pragma unroll
        for (int q = 0; q < kGMaxDPT; ++q) {
          tot[q] += Elt<E>::round(acc[q]);
          acc[q] = 0.f;
        }
        chunk_end += a.chunk;
      }
      const float pj = ps[j];
      const E* wrow = Wm + (base + j) * a.D;
#pragma unroll
      for (int q = 0; q < kGMaxDPT; ++q) {
        const int64_t dcol = tid + static_cast<int64_t>(q) * kGT;
        if (q < nd && dcol < a.D) acc[q] = fmaf(pj, Elt<E>::load(wrow + dcol), acc[q]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < kGMaxDPT; ++q) tot[q] += EMU ? Elt<E>::round(acc[q]) : acc[q];

  // ---- per-token reductions and the den division (v41:579-586)
  const float G = block_sum<kGT>(gsum, red);
  const float I = block_sum<kGT>(isum, red);
  const float NA = block_sum<kGT>(nact, red);
  const float den = fmaxf(V401 ? G : I, 1.0f);
  E* O = static_cast<E*>(a.out) + tr * a.D;
#pragma unroll
  for (int q = 0; q < kGMaxDPT; ++q) {
    const int64_t dcol = tid + static_cast<int64_t>(q) * kGT;
    if (q < nd && dcol < a.D) {
      const float v = Elt<E>::round(tot[q] / den);
      Elt<E>::store(O + dcol, v * a.scale);
    }
  }
  float dg[SRW_TDIAG_COUNT];
  if (DIAG) {
    dg[SRW_TDIAG_S_MEAN] = s_mean;
    dg[SRW_TDIAG_S_STD] = s_std;
    dg[SRW_TDIAG_TAU] = tau;
    dg[SRW_TDIAG_SUM_S3] = m3;
    dg[SRW_TDIAG_SUM_S4] = m4;
    dg[SRW_TDIAG_GATE_MAX] = block_max<kGT>(gmax, red);
    dg[SRW_TDIAG_INT_SUM] = I;
    dg[SRW_TDIAG_N_STRONG] = block_sum<kGT>(nstrong, red);
    dg[SRW_TDIAG_N_BOUNDARY] = block_sum<kGT>(nbound, red);
    dg[SRW_TDIAG_N_BAND075] = block_sum<kGT>(n075, red);
    dg[SRW_TDIAG_N_BAND030] = block_sum<kGT>(n030, red);
    dg[SRW_TDIAG_G_LOG_G] = block_sum<kGT>(glogg, red);
    dg[SRW_TDIAG_INT_MAX] = block_max<kGT>(imax, red);
    dg[SRW_TDIAG_N_INT_CAP] = block_sum<kGT>(ncap, red);
  }
  if (tid == 0) {
    if (a.gate_sum) a.gate_sum[tr] = G;
    if (a.den) a.den[tr] = den;
    if (a.n_active) a.n_active[tr] = static_cast<int32_t>(NA);
    if (DIAG && a.token_diag) {
      for (int k = 0; k < SRW_TDIAG_COUNT; ++k) a.token_diag[tr * SRW_TDIAG_COUNT + k] = dg[k];
    }
  }
}

// r / (||r|| + 1e-8) per row, in the storage dtype (v401:300-301 bf16,
// v401:1456-1457 f32).  One workgroup per row.
template <typename E>
__global__ __launch_bounds__(kGT) void normalize_rows_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                             int64_t D) {
  __shared__ float red[kGT / kWave];
  const E* row = src + static_cast<int64_t>(blockIdx.x) * D;
  E* orow = dst + static_cast<int64_t>(blockIdx.x) * D;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < D; i += kGT) {
    const float v = Elt<E>::load(row + i);
    ss += v * v;
  }
  const float nrm = sqrtf(block_sum<kGT>(ss, red));
  // bf16: norm rounded to bf16, +1e-8 in bf16, elementwise bf16 division
  const float denom = Elt<E>::round(Elt<E>::round(nrm) + 1e-8f);
  for (int64_t i = threadIdx.x; i < D; i += kGT) Elt<E>::store(orow + i, Elt<E>::load(row + i) / denom);
}

__global__ void fill_kernel(float* p, int64_t n, float v) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = v;
}

template <typename E, bool V401, bool EMU, bool DIAG>
hipError_t launch_generic(const GenericParams& p, int64_t blocks, size_t smem, hipStream_t s) {
  dominant_kernel_begin(s);
  hipLaunchKernelGGL((srw_generic_kernel<E, V401, EMU, DIAG>), dim3(static_cast<unsigned>(blocks)), dim3(kGT),
                     smem, s, p);
  dominant_kernel_end(s);
  return hipGetLastError();
}

template <typename E>
hipError_t generic_forward_t(const LaunchArgs& a) {
  const srw_desc_t& d = a.d;
  const bool v401 = d.gate == SRW_GATE_GELU_V401;
  const bool emu = (d.flags & SRW_FLAG_EMULATE) != 0;
  const bool diag = (d.flags & SRW_FLAG_DIAG) != 0;
  GenericParams p{};
  p.x = a.in.x;
  p.h = a.in.h;
  p.emb = a.in.emb;
  p.tau_off = a.in.tau_offset;
  p.read = a.in.read;
  p.write = a.in.write;
  p.out = a.o.out;
  p.gate_sum = a.o.gate_sum;
  p.den = a.o.den;
  p.n_active = a.o.n_active;
  p.pass_mask = a.o.pass_mask;
  p.token_diag = a.o.token_diag;
  p.unit_diag = a.o.unit_diag;
  p.gate_out = a.o.gate;
  p.D = d.d_model;
  p.dr = d.d_route;
  p.N = d.n_units;
  p.words = a.words;
  p.chunk = a.chunk;
  p.R = d.n_routes;
  p.stats = d.stats_mode;
  p.gp = a.gp;
  p.scale = d.scale;

  hipError_t e = hipSuccess;
  if (v401) {
    // forward-normalised copies of R and W live in the workspace
    E* rn = reinterpret_cast<E*>(a.ws);
    E* wn = rn + d.n_units * d.d_model;
    hipLaunchKernelGGL((normalize_rows_kernel<E>), dim3(static_cast<unsigned>(d.n_units)), dim3(kGT), 0,
                       a.stream, static_cast<const E*>(a.in.read), rn, d.d_model);
    hipLaunchKernelGGL((normalize_rows_kernel<E>), dim3(static_cast<unsigned>(d.n_units)), dim3(kGT), 0,
                       a.stream, static_cast<const E*>(a.in.write), wn, d.d_model);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    p.read = rn;
    p.write = wn;
  }
  if (diag && a.o.unit_diag) {
    if ((e = fill_f32(a.o.unit_diag, d.n_units * SRW_UDIAG_COUNT, 0.f, a.stream)) != hipSuccess) return e;
  }
  const int64_t blocks = d.T * d.n_routes;
  const size_t smem = static_cast<size_t>(d.d_route + d.d_model + kGT + kGT / kWave) * sizeof(float);
  if (v401) {
    if (emu) return diag ? launch_generic<E, true, true, true>(p, blocks, smem, a.stream)
                         : launch_generic<E, true, true, false>(p, blocks, smem, a.stream);
    return diag ? launch_generic<E, true, false, true>(p, blocks, smem, a.stream)
                : launch_generic<E, true, false, false>(p, blocks, smem, a.stream);
  }
  if (emu) return diag ? launch_generic<E, false, true, true>(p, blocks, smem, a.stream)
                       : launch_generic<E, false, true, false>(p, blocks, smem, a.stream);
  return diag ? launch_generic<E, false, false, true>(p, blocks, smem, a.stream)
              : launch_generic<E, false, false, false>(p, blocks, smem, a.stream);
}

}  // namespace

// The same per row for bf16 with one wave per row (four rows a workgroup):
// the pools' rows are short (D <= 4096), and a workgroup per row leaves most
// of its threads idle.
__global__ __launch_bounds__(256) void normalize_rows_wave_kernel(const bf16_t* __restrict__ src,
                                                                  bf16_t* __restrict__ dst, int64_t N, int64_t D) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= N) return;
  const int lane = threadIdx.x & 63;
  const bf16_t* row = src + r * D;
  bf16_t* orow = dst + r * D;
  float ss = 0.f;
  for (int64_t i = lane; i < D; i += 64) {
    const float v = Elt<bf16_t>::load(row + i);
    ss += v * v;
  }
  const float nrm = sqrtf(wave_sum(ss));
  const float denom = Elt<bf16_t>::round(Elt<bf16_t>::round(nrm) + 1e-8f);
  for (int64_t i = lane; i < D; i += 64) Elt<bf16_t>::store(orow + i, Elt<bf16_t>::load(row + i) / denom);
}

hipError_t normalize_rows_bf16(const uint16_t* src, uint16_t* dst, int64_t N, int64_t D, hipStream_t s) {
  if (N <= 0) return hipSuccess;
  hipLaunchKernelGGL(normalize_rows_wave_kernel, dim3(static_cast<unsigned>((N + 3) / 4)), dim3(256), 0, s,
                     reinterpret_cast<const bf16_t*>(src), reinterpret_cast<bf16_t*>(dst), N, D);
  return hipGetLastError();
}

hipError_t normalize_rows_f32(const float* src, float* dst, int64_t N, int64_t D, hipStream_t s) {
  if (N <= 0) return hipSuccess;
  hipLaunchKernelGGL((normalize_rows_kernel<float>), dim3(static_cast<unsigned>(N)), dim3(kGT), 0, s, src, dst, D);
  return hipGetLastError();
}

hipError_t fill_f32(float* p, int64_t n, float v, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

size_t generic_workspace_bytes(const srw_desc_t& d) {
  if (d.gate != SRW_GATE_GELU_V401) return 0;
  const size_t elt = d.dtype == SRW_BF16 ? 2 : 4;
  return 2 * static_cast<size_t>(d.n_units) * static_cast<size_t>(d.d_model) * elt;
}

bool generic_supports(const srw_desc_t& d) {
  if (d.d_model > static_cast<int64_t>(kGT) * kGMaxDPT) return false;
  // LDS: h row + x row + staging, within the 64 KiB default dynamic limit
  const int64_t lds = (d.d_route + d.d_model + kGT + kGT / kWave) * 4;
  return lds <= 64 * 1024;
}

hipError_t generic_forward(const LaunchArgs& a) {
  if (a.d.dtype == SRW_BF16) return generic_forward_t<bf16_t>(a);
  return generic_forward_t<float>(a);
}

}  // namespace srw

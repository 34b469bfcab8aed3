// srw_gram.hip -- per-token score moments from the pool's Gram matrix
// (SRW_STATS_GRAM).
//
// The reference's pass 1 (models/dawn_spatial_v41_exp.py:433-462) runs the
// full score GEMM h.E^T only to get, per token, sum_n s and sum_n s^2.  Both
// are quadratic forms of h with token-independent pool statistics:
//
//   sum_n s_n   = h . esum,          esum = sum_n e_n            [d_route]
//   sum_n s_n^2 = h^T G h,           G    = E^T E                [d_route^2]
//
// so this path costs 2 N dr^2 + 2 T dr^2 flops instead of 2 T N dr.  The
// moments are those of the unrounded fp32 scores (the reference rounds each
// score to bf16 first); the difference moves tau by ~1e-5 relative, far
// below a bf16 score ulp.
//
// Kernels:
//   gram        split-K syrk on the matrix cores: partial G over a range of
//               32-unit tiles, from E packed unit-contiguous (the same
//               fragment layout as the packed W^T of the write GEMM, so one
//               fragment serves as the A or the B operand); also partial
//               esum from the fragments' own values.
//   gram_reduce sums the split-K partials; emits G as hi + lo bf16 fragments
//               (G = hi + lo to ~2^-16 relative) for the token GEMM, and esum.
//   gram_mom    per (128 tokens, 32-row block of G): U^T = G_blk . H^T on the
//               matrix cores, sum_n U^T[n][t] h[t][n] -> partial sum s^2; the
//               first block also writes h . esum.  Output: the main kernel's
//               moment partials mom[DB_r][T][2].

#include "srw_internal.hpp"

namespace srw {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kFrag = 512;        // bf16 elements per operand fragment
constexpr int kFragBytes = 1024;
constexpr int kGramSplits = 28;   // split-K factor of the syrk

__device__ inline f32x16_t mfma(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ inline uint32_t pack_bf16(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ inline float lo_f32(uint32_t p) { return __uint_as_float(p << 16); }
__device__ inline float hi_f32(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }
__device__ inline int acc_row(int v, int half) { return 8 * (v >> 2) + 4 * half + (v & 3); }

// region = RB x RB blocks of 32 x 32; the 4 waves of a workgroup split it
// into (RB/2) x (RB/2)-block quadrants (RB >= 2) or wave 0 does it (RB == 1).
struct GramParams {
  const uint16_t* ep;   // packed E fragments [ntiles][DBr][2][64][8]
  float* gpart;         // [KS][dr][dr]
  float* epart;         // [KS][dr]
  int ntiles, DBr, RB, KS;
};

__global__ __launch_bounds__(256) void gram_kernel(GramParams p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, col = lane & 31;
  // G is symmetric: only the regions rr <= rc are computed
  const int NR = p.DBr / p.RB, NU = NR * (NR + 1) / 2;
  const int region = blockIdx.x % NU, ks = blockIdx.x / NU;
  int rr = 0, rem = region;
  while (rem >= NR - rr) {
    rem -= NR - rr;
    ++rr;
  }
  const int rc = rr + rem;
  const int k0 = static_cast<int>(static_cast<int64_t>(p.ntiles) * ks / p.KS);
  const int k1 = static_cast<int>(static_cast<int64_t>(p.ntiles) * (ks + 1) / p.KS);
  // fragments per tile staged in LDS: A blocks (rows) then B blocks (cols), 2 k-steps each
  const int nfa = 2 * p.RB, nf = 4 * p.RB;
  const int stage = nf * kFragBytes;
  // this wave's blocks within the region
  const int QB = p.RB >= 2 ? p.RB / 2 : 1;          // blocks per wave side
  const bool active = p.RB >= 2 || wave == 0;
  const int wa = p.RB >= 2 ? (wave >> 1) * QB : 0;  // first row block (in region)
  const int wb = p.RB >= 2 ? (wave & 1) * QB : 0;   // first col block (in region)

  auto issue = [&](int tile, int st) {
    for (int f = wave; f < nf; f += 4) {
      const int side = f < nfa ? 0 : 1;
      const int ff = side ? f - nfa : f;
      const int blk = (side ? rc : rr) * p.RB + (ff >> 1);
      const int j = ff & 1;
      const uint16_t* src = p.ep + ((static_cast<int64_t>(tile) * p.DBr + blk) * 2 + j) * kFrag + lane * 8;
      __builtin_amdgcn_global_load_lds(src, (lds_ptr_t)(lds + st * stage + f * kFragBytes), 16, 0, 0);
    }
  };

  f32x16_t acc[2][2];
  for (int a = 0; a < 2; ++a)
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x16_t{};
  float es[2] = {0.f, 0.f};
  if (k0 < k1) issue(k0, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  for (int tile = k0; tile < k1; ++tile) {
    const int st = (tile - k0) & 1;
    if (tile + 1 < k1) issue(tile + 1, st ^ 1);
    if (active) {
      const char* base = lds + st * stage + lane * 16;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        u32x4_t A[2], B[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (q < QB) {
            A[q] = *reinterpret_cast<const u32x4_t*>(base + (2 * (wa + q) + j) * kFragBytes);
            B[q] = *reinterpret_cast<const u32x4_t*>(base + (nfa + 2 * (wb + q) + j) * kFragBytes);
          }
        }
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            if (a < QB && b < QB) acc[a][b] = mfma(A[a], B[b], acc[a][b]);
        // column sums of E for esum: the diagonal regions' left waves
        if (rr == rc && wb == 0) {
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            if (q < QB) {
#pragma unroll
              for (int e = 0; e < 4; ++e) es[q] += lo_f32(A[q][e]) + hi_f32(A[q][e]);
            }
          }
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
  }
  if (!active) return;
  const int dr = p.DBr * 32;
  float* g = p.gpart + static_cast<int64_t>(ks) * dr * dr;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (a < QB && b < QB) {
        const int ib = rr * p.RB + wa + a, jb = rc * p.RB + wb + b;
#pragma unroll
        for (int v = 0; v < 16; ++v) g[(32 * ib + acc_row(v, half)) * dr + 32 * jb + col] = acc[a][b][v];
      }
    }
  if (rr == rc && wb == 0) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (q < QB) {
        const float s = es[q] + __shfl_xor(es[q], 32);
        if (half == 0) p.epart[static_cast<int64_t>(ks) * dr + 32 * (rr * p.RB + wa + q) + col] = s;
      }
    }
  }
}

// G (and esum) from the partials, read coalesced (one thread per G element,
// consecutive threads along a row); G is written as the token GEMM's
// A-operand fragments Gp[nb][ks][hl][lane][8] = {hi, lo}(G[32 nb + lane % 32][16 ks + 8 (lane / 32) + i]).
template <int KS>
__global__ __launch_bounds__(256) void gram_reduce_kernel(const float* __restrict__ gpart,
                                                          const float* __restrict__ epart, uint16_t* __restrict__ gp,
                                                          float* __restrict__ esum, int dr, int RB) {
  const int64_t total = static_cast<int64_t>(dr) * dr;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int row = static_cast<int>(idx / dr), colk = static_cast<int>(idx % dr);
    // lower-triangle regions were not computed: read the transposed element
    const bool mirror = row / (32 * RB) > colk / (32 * RB);
    const int64_t src = mirror ? static_cast<int64_t>(colk) * dr + row : idx;
    float part[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) part[s] = gpart[static_cast<int64_t>(s) * total + src];
    float gsum = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) gsum += part[s];
    const float hi = round_bf16(gsum);
    const float lo = gsum - hi;
    const int nb = row >> 5, ks = colk >> 4;
    const int lane = (row & 31) + 32 * ((colk >> 3) & 1), i = colk & 7;
    const int64_t fr = static_cast<int64_t>(nb) * (dr / 16) + ks;
    const int64_t base = ((fr * 2) * 64 + lane) * 8 + i;
    gp[base] = f32_to_bf16_bits(hi);
    gp[base + 64 * 8] = f32_to_bf16_bits(lo);
    if (idx < dr) {
      float e = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s) e += epart[static_cast<int64_t>(s) * dr + idx];
      esum[idx] = e;
    }
  }
}

struct GramMaskPrep {
  uint32_t* mask32;  // pass mask as 32-bit words, or null
  int64_t words32, cs;
  int nc, ntiles;
};

// One workgroup per (128 tokens, 32-row block nb of G): the block's hi/lo
// fragments are staged once in LDS and shared by the four waves, each of which
// owns 32 tokens.  mom[nb][t] = (nb == 0 ? h.esum : 0, sum_{n in block} (G h)_n h_n).
template <int KH>
__global__ __launch_bounds__(256) void gram_mom_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ gp,
                                                       const float* __restrict__ esum, float* __restrict__ mom,
                                                       int64_t T, GramMaskPrep mp) {
  constexpr int DR = KH * 16, DBr = DR / 32;
  __shared__ __attribute__((aligned(16))) uint16_t gs[KH * 2 * kFrag];
  const int lane = threadIdx.x & 63, half = lane >> 5, col = lane & 31, wave = threadIdx.x >> 6;
  const int nb = static_cast<int>(blockIdx.x % DBr);
  const int64_t t0 = (blockIdx.x / DBr) * 128 + 32 * wave;
  const u32x4_t* gsrc = reinterpret_cast<const u32x4_t*>(gp) + static_cast<int64_t>(nb) * KH * 2 * 64;
  for (int i = threadIdx.x; i < KH * 2 * 64; i += 256) reinterpret_cast<u32x4_t*>(gs)[i] = gsrc[i];
  __syncthreads();
  if (t0 >= T) return;
  const int64_t t = t0 + col;
  const int64_t tl = t < T ? t : T - 1;
  const uint16_t* hrow = h + tl * DR;
  const u32x4_t* g = reinterpret_cast<const u32x4_t*>(gs) + lane;
  f32x16_t acc = {};
#pragma unroll
  for (int ks = 0; ks < KH; ++ks) {
    const u32x4_t hb = *reinterpret_cast<const u32x4_t*>(hrow + 16 * ks + 8 * half);
    acc = mfma(g[(ks * 2) * 64], hb, acc);       // G hi
    acc = mfma(g[(ks * 2 + 1) * 64], hb, acc);   // G lo
  }
  // acc[v] = (G h_t)[32 nb + acc_row(v, half)]
  float s2 = 0.f;
#pragma unroll
  for (int v = 0; v < 16; ++v) s2 += acc[v] * bf16_to_f32(hrow[32 * nb + acc_row(v, half)]);
  s2 += __shfl_xor(s2, 32);
  float s1 = 0.f;
  if (nb == 0) {
    // h . esum, eight elements per step; each lane-half takes half the row
    for (int k = half * (DR / 2); k < (half + 1) * (DR / 2); k += 8) {
      const u32x4_t hv = *reinterpret_cast<const u32x4_t*>(hrow + k);
      const float4 e0 = *reinterpret_cast<const float4*>(esum + k);
      const float4 e1 = *reinterpret_cast<const float4*>(esum + k + 4);
      s1 += lo_f32(hv[0]) * e0.x + hi_f32(hv[0]) * e0.y + lo_f32(hv[1]) * e0.z + hi_f32(hv[1]) * e0.w;
      s1 += lo_f32(hv[2]) * e1.x + hi_f32(hv[2]) * e1.y + lo_f32(hv[3]) * e1.z + hi_f32(hv[3]) * e1.w;
    }
    s1 += __shfl_xor(s1, 32);
    // pass-mask words the main kernel ORs into, and the unused upper half of the last word
    if (mp.mask32 && half == 0 && t < T) {
      for (int c = 1; c < mp.nc; ++c) {
        const int64_t b = c * mp.cs;
        if (b % 32) mp.mask32[t * mp.words32 + b / 32] = 0u;
      }
      if (mp.ntiles & 1) mp.mask32[t * mp.words32 + mp.ntiles] = 0u;
    }
  }
  if (half == 0 && t < T) {
    float* m = mom + (static_cast<int64_t>(nb) * T + t) * 2;
    m[0] = s1;
    m[1] = s2;
  }
}

size_t al(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

}  // namespace

bool gram_supports(int64_t dr) { return dr == 384 || dr == 128 || dr == 64 || dr == 32; }

int gram_moment_parts(int64_t dr) { return static_cast<int>(dr / 32); }

size_t gram_workspace_bytes(int64_t N, int64_t dr) {
  const int64_t ntiles = (N + 31) / 32;
  return al(static_cast<size_t>(ntiles) * 32 * dr * 2) + al(static_cast<size_t>(kGramSplits) * dr * dr * 4) +
         al(static_cast<size_t>(kGramSplits) * dr * 4) + al(static_cast<size_t>(dr) * dr * 2 * 2) +
         al(static_cast<size_t>(dr) * 4);
}

hipError_t gram_moments(const uint16_t* emb, const uint16_t* h, int64_t T, int64_t N, int64_t dr, float* mom,
                        char* ws, hipStream_t s, uint32_t* mask32, int64_t words32, int64_t cs, int nc,
                        bool pool_cached) {
  const int64_t ntiles = (N + 31) / 32;
  const int DBr = static_cast<int>(dr / 32);
  char* p = ws;
  uint16_t* ep = reinterpret_cast<uint16_t*>(p);
  p += al(static_cast<size_t>(ntiles) * 32 * dr * 2);
  float* gpart = reinterpret_cast<float*>(p);
  p += al(static_cast<size_t>(kGramSplits) * dr * dr * 4);
  float* epart = reinterpret_cast<float*>(p);
  p += al(static_cast<size_t>(kGramSplits) * dr * 4);
  uint16_t* gp = reinterpret_cast<uint16_t*>(p);
  p += al(static_cast<size_t>(dr) * dr * 2 * 2);
  float* esum = reinterpret_cast<float*>(p);
  hipError_t e;
  GramMaskPrep mp{mask32, words32, cs, nc, static_cast<int>(ntiles)};
  if (!pool_cached) {  // else G and esum of this pool are already in the workspace
    if ((e = pack_unit_major(emb, ep, N, static_cast<int>(dr), s)) != hipSuccess) return e;

    GramParams gpp{};
    gpp.ep = ep;
    gpp.gpart = gpart;
    gpp.epart = epart;
    gpp.ntiles = static_cast<int>(ntiles);
    gpp.DBr = DBr;
    gpp.RB = DBr >= 4 ? 4 : DBr;
    gpp.KS = kGramSplits;
    const int NR = DBr / gpp.RB, NU = NR * (NR + 1) / 2;
    const size_t smem = static_cast<size_t>(2 * 4 * gpp.RB) * kFragBytes;
    if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(gram_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 static_cast<int>(smem))) != hipSuccess)
      return e;
    hipLaunchKernelGGL(gram_kernel, dim3(static_cast<unsigned>(NU * kGramSplits)), dim3(256), smem, s, gpp);
    if ((e = hipGetLastError()) != hipSuccess) return e;

    int64_t blocks = (dr * dr + 255) / 256;
    hipLaunchKernelGGL(gram_reduce_kernel<kGramSplits>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, gpart,
                       epart, gp, esum, static_cast<int>(dr), gpp.RB);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }

  const unsigned mblocks = static_cast<unsigned>(((T + 127) / 128) * DBr);
  switch (dr) {
    case 384: hipLaunchKernelGGL(gram_mom_kernel<24>, dim3(mblocks), dim3(256), 0, s, h, gp, esum, mom, T, mp); break;
    case 128: hipLaunchKernelGGL(gram_mom_kernel<8>, dim3(mblocks), dim3(256), 0, s, h, gp, esum, mom, T, mp); break;
    case 64: hipLaunchKernelGGL(gram_mom_kernel<4>, dim3(mblocks), dim3(256), 0, s, h, gp, esum, mom, T, mp); break;
    case 32: hipLaunchKernelGGL(gram_mom_kernel<2>, dim3(mblocks), dim3(256), 0, s, h, gp, esum, mom, T, mp); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

}  // namespace srw

// srw_tiled_f32.hip -- fp32 SRW forward on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32): the dtype-preserving fp32 `_srw_inference`
// (v41:1713-1738: centred two-pass statistics, one chunk), and fp32 calls
// with one-pass statistics -- an extension with no reference counterpart
// (the reference's fused_gate_srw casts every operand to bf16, v41:422-428),
// checked against this library's scalar kernels only; in fp32 the chunk
// plan changes no rounding (every chunk's partial write GEMM stays fp32).
//
// The layer runs as the bf16 tiled family does (srw_tiled.hip), with every
// operand and intermediate in fp32:
//
//   pack   W [N, D] -> W^T [D, N64] (unit-contiguous rows, zero tail)
//   stats  S = E.H^T per 256-unit x 256-token tile, stored as S [T, N64]
//          fp32 (v41:1717-1718); per token and 128 units: sum s and sum
//          s^2, or (centred statistics) sum (s - their mean)^2 from the
//          registers, which the tau kernel merges into the row's centred
//          sum of squares (v41:1719-1721) without a second pass over S
//   gate   per tile XR = R.X^T, the v4.1 gate of the stored scores in the
//          reference's fp32 expression order (v41:1723-1728), P = gate * xr
//          over S in place (v41:1735); per-token
//          sum gate, sum intensity, active count, and the pass bits
//   write  OUT = P . W over N-splits of the units, fp32 partials
//   final  out = sum of the partials / max(sum intensity, 1) * scale in fp32
//          (v41:1736-1737)
//
// The GEMM main loop (fgemm_loop): an output tile of 32 GA x 32 GB per
// workgroup of 4 waves (256 units x 64 tokens in the score and gate kernels,
// 128 tokens x 192 or 256 x 256 columns in the write kernel), operands
// K-contiguous in memory, 32-wide k blocks (one 128-byte line per row) in a
// double-buffered LDS ring filled by direct global->LDS loads, 16-byte
// pieces XOR-swizzled by row.  In the 32 x 32 x 2 MFMA the lanes of half h supply k index h of the
// step; here step s of a k block takes k = s from half 0 and k = 16 + s from
// half 1 (any assignment of k to (step, half) shared by both operands gives
// the same sum), so a lane's 16 steps read 64 contiguous bytes of its row:
// four 16-byte LDS reads per operand row block.

#include "srw_internal.hpp"
#include "srw_mfma_util.hpp"

namespace srw {

namespace {

constexpr int kFThreads = 256;              // 4 waves
constexpr int kFRows = 256;                 // rows per operand tile = output tile side
constexpr int kFK = 32;                     // fp32 k per stage: one 128-byte line per row
constexpr int kFOpBytes = kFRows * kFK * 4;  // 32 KB
constexpr int kFStageBytes = 2 * kFOpBytes;  // A and B tiles
constexpr int kFGemmLds = 2 * kFStageBytes;  // two stages: 128 KB
constexpr int kFGroupBytes = 32 * kFK * 4;   // 32 rows: one MFMA operand's rows
constexpr int kFNAlign = 64;                 // padding of the stored [., N] rows

__device__ inline f32x16_t mfma_f32(float a, float b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// An operand tile in LDS: 32-row groups of 4 KB; row u of a group at
// (u / 8) * 1 KB + (u % 8) * 128 B, its 16-byte piece q in slot q ^ fswz(u).
__device__ inline int fswz(int u) { return (u & 7) ^ ((u >> 3) & 1); }

// The G rows a wave loads per stage: rows 32 i + 8 wave + lane / 8 of the
// tile (i = 0..G-1, one per 32-row group), 16 bytes each per lane.  Memory row of tile row r =
// min(row0 + r, rows - 1) / div (div = 2 maps paired-route rows to x rows).
template <int G>
struct FOpnd {
  const char* base;  // byte address of memory row row0 / div, k = 0 (uniform)
  uint32_t off[G];   // per-lane byte offsets from base: row and swizzled piece
};

template <int G = 8>
__device__ inline FOpnd<G> make_fopnd(const float* p, int64_t ld, int64_t row0, int64_t rows, int div, int wave,
                                      int lane) {
  FOpnd<G> o;
  const int64_t base_row = row0 / div;
  o.base = reinterpret_cast<const char*>(p + base_row * ld);
  const int r8 = lane >> 3;
  const int piece = (lane & 7) ^ r8 ^ (wave & 1);  // fswz(8 wave + r8) = r8 ^ (wave & 1)
#pragma unroll
  for (int i = 0; i < G; ++i) {
    int64_t row = row0 + 32 * i + 8 * wave + r8;
    row = row < rows ? row : rows - 1;
    o.off[i] = static_cast<uint32_t>(((row / div - base_row) * ld + 4 * piece) * 4);
  }
  return o;
}

// acc[i][j] += A-tile rows (32 (ga0 + i) ..) . B-tile rows (32 (gb0 + j) ..)^T
// over k in [k0, k0 + 32 nk), for an A tile of GA 32-row groups and a B tile
// of GB groups (a stage holds both: (GA + GB) x 4 KB); the wave's accumulator
// block is MI x MJ MFMA tiles at groups (ga0, gb0).
//
// Per k block: 16 steps of MI x MJ MFMAs in two halves (steps 0-7: pieces 4 h,
// 4 h + 1 of each row; steps 8-15: pieces 4 h + 2, 4 h + 3).  A half's
// fragments are read while the other half's MFMAs run: the second half of
// block kb under the first half's MFMAs, the first half of block kb + 1
// under the second half's.  Between the two halves the workgroup barrier
// that ends the reads of block kb's stage, the loads of block kb + 2 into
// it, and the wait for block kb + 1 (loaded one block earlier).
template <int GA, int GB, int MI, int MJ>
__device__ inline void fgemm_loop(f32x16_t (&acc)[MI][MJ], const FOpnd<GA>& A, const FOpnd<GB>& B, int64_t k0,
                                  int nk, char* lds, int ga0, int gb0, int wave, int lane) {
  constexpr int kOpA = GA * kFGroupBytes, kStage = (GA + GB) * kFGroupBytes;
  static_assert(2 * kStage <= kFGemmLds, "two stages fit the LDS allocation");
  static_assert(GA + GB <= 63, "loads per block within the vmcnt range");
  const int u = lane & 31, h = lane >> 5;
  int le[4];  // piece 4 h + m of row u
#pragma unroll
  for (int m = 0; m < 4; ++m) le[m] = (u >> 3) * 1024 + (u & 7) * 128 + (((4 * h + m) ^ fswz(u)) * 16);
  // block b's GA + GB loads per thread: one piece per 32-row group
  auto issue = [&](int b, char* stage) {
    const int64_t kbyte = (k0 + static_cast<int64_t>(b) * kFK) * 4;
#pragma unroll
    for (int q = 0; q < GA; ++q) g2lds16(A.base + kbyte + A.off[q], stage + q * kFGroupBytes + wave * 1024);
#pragma unroll
    for (int q = 0; q < GB; ++q) g2lds16(B.base + kbyte + B.off[q], stage + kOpA + q * kFGroupBytes + wave * 1024);
  };
  // half hf of block kb's fragments: 8 floats a lane per row block of A (B)
  auto read = [&](const char* st, int hf, float (&fa)[MI][8], float (&fb)[MJ][8]) {
#pragma unroll
    for (int g = 0; g < MI; ++g) {
      const char* ra = st + (ga0 + g) * kFGroupBytes;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const float4 qa = *reinterpret_cast<const float4*>(ra + le[2 * hf + m]);
        fa[g][4 * m] = qa.x;
        fa[g][4 * m + 1] = qa.y;
        fa[g][4 * m + 2] = qa.z;
        fa[g][4 * m + 3] = qa.w;
      }
    }
#pragma unroll
    for (int g = 0; g < MJ; ++g) {
      const char* rb = st + kOpA + (gb0 + g) * kFGroupBytes;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const float4 qb = *reinterpret_cast<const float4*>(rb + le[2 * hf + m]);
        fb[g][4 * m] = qb.x;
        fb[g][4 * m + 1] = qb.y;
        fb[g][4 * m + 2] = qb.z;
        fb[g][4 * m + 3] = qb.w;
      }
    }
  };
  auto steps = [&](const float (&fa)[MI][8], const float (&fb)[MJ][8]) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int q = 0; q < MI * MJ; ++q)
        acc[q / MJ][q % MJ] = mfma_f32(fa[q / MJ][s], fb[q % MJ][s], acc[q / MJ][q % MJ]);
  };
  // block kb has landed in every wave's share (kb + 1 the last block issued)
  auto landed = [&](int kb) {
    constexpr int kN = GA + GB;  // loads of block kb + 1, still in flight
    if (kb + 1 < nk)
      __builtin_amdgcn_s_waitcnt(0x0F70 | (kN & 0xF) | ((kN >> 4) << 14));  // vmcnt(GA + GB)
    else
      wait_vm0();
    barrier_lds();
  };
  float fa0[MI][8], fb0[MJ][8], fa1[MI][8], fb1[MJ][8];
  issue(0, lds);
  if (nk > 1) issue(1, lds + kStage);
  landed(0);
  read(lds, 0, fa0, fb0);
  for (int kb = 0; kb < nk; ++kb) {
    char* st = lds + (kb & 1) * kStage;
    read(st, 1, fa1, fb1);
    steps(fa0, fb0);
    barrier_lds();  // no wave reads block kb's stage any more
    if (kb + 2 < nk) issue(kb + 2, st);
    if (kb + 1 < nk) {
      landed(kb + 1);
      read(lds + ((kb + 1) & 1) * kStage, 0, fa0, fb0);
    }
    steps(fa1, fb1);
  }
}

// Workgroup -> (row tile, column tile) with the column tile shared by the
// workgroups of one XCD (blockIdx % 8): they walk the row tiles of one column
// tile together, so its operand rows are fetched into that XCD's L2 once.
__device__ inline bool ftile_of(int nrow, int ncol, int& rt, int& ct) {
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  ct = (k / nrow) * 8 + x;
  rt = k % nrow;
  return ct < ncol;
}

// ---------------------------------------------------------------------------
// pack: W [N, D] -> W^T [D, N64], zero for units >= N
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_wt_f32_kernel(const float* __restrict__ W, float* __restrict__ WT,
                                                          int64_t N, int64_t N64, int D) {
  __shared__ float tile[64][65];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int d0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t n = n0 + r;
    const int d = d0 + tx;
    tile[r][tx] = (n < N && d < D) ? W[n * D + d] : 0.f;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int d = d0 + r;
    const int64_t n = n0 + tx;
    if (d < D && n < N64) WT[static_cast<int64_t>(d) * N64 + n] = tile[tx][r];
  }
}

// ---------------------------------------------------------------------------
// stats: the fp32 scores of a tile, stored, and per-token moment partials
// ---------------------------------------------------------------------------
struct FStatsParams {
  const float* h;    // [Tv, dr]
  const float* emb;  // [N, dr]
  float* S;          // [Tv, N64] fp32 scores (zero for units >= N)
  float* mom;        // [2 CT][Tv][2]: per 128 units (sum s, sum s^2), or (sum s, sum (s - their mean)^2)
  int64_t Tv, N, N64, dr;
  int RT, CT;    // token tiles, unit tiles
  int centred;   // second moments about the 128 units' own mean (merged by srw_tau_kernel's kTauChan)
};

// A workgroup takes 256 units x 64 MJ tokens (2 x 2 waves of 128 units x
// 32 MJ tokens).  The launches use MJ = 1: 80 KB of LDS and ~180 registers a
// wave, so two workgroups share a CU and one's epilogue (the moments and
// score stores here, the gate and P stores in f32_gate_kernel) runs beside
// the other's MFMAs -- a wave's own VALU work does not overlap its MFMAs.
// (256-token tiles, MJ = 4, one workgroup per CU: 5% slower per call.)
template <int MJ>
__global__ __launch_bounds__(kFThreads, 1) void f32_stats_kernel(FStatsParams p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wa = wave >> 1, wb = wave & 1, u = lane & 31, h = lane >> 5;
  int rt, ct;
  if (!ftile_of(p.RT, p.CT, rt, ct)) return;
  const int64_t u0 = static_cast<int64_t>(ct) * kFRows, v0 = static_cast<int64_t>(rt) * 64 * MJ;
  const FOpnd<8> A = make_fopnd<8>(p.emb, p.dr, u0, p.N, 1, wave, lane);
  const FOpnd<2 * MJ> B = make_fopnd<2 * MJ>(p.h, p.dr, v0, p.Tv, 1, wave, lane);
  f32x16_t acc[4][MJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc[i][j] = f32x16_t{};
  fgemm_loop(acc, A, B, 0, static_cast<int>(p.dr / kFK), lds, 4 * wa, MJ * wb, wave, lane);

  // element v of accumulator (i, j): unit 128 wa + 32 i + 8 (v / 4) + 4 h + v % 4
  // of the tile, token 32 (MJ wb + j) + u
  const int64_t nleft = p.N - (u0 + 128 * wa + 4 * h);  // units of this wave-row left in the pool
#pragma unroll
  for (int j = 0; j < MJ; ++j) {
    const int64_t t = v0 + 32 * (MJ * wb + j) + u;
    float* srow = p.S + (t < p.Tv ? t : 0) * p.N64;
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int v = 0; v < 16; v += 4) {
        const int r = 32 * i + 8 * (v >> 2);  // unit offset from u0 + 128 wa + 4 h
        float4 q;
        q.x = r < nleft ? acc[i][j][v] : 0.f;
        q.y = r + 1 < nleft ? acc[i][j][v + 1] : 0.f;
        q.z = r + 2 < nleft ? acc[i][j][v + 2] : 0.f;
        q.w = r + 3 < nleft ? acc[i][j][v + 3] : 0.f;
        s1 += q.x;
        s2 += q.x * q.x;
        s1 += q.y;
        s2 += q.y * q.y;
        s1 += q.z;
        s2 += q.z * q.z;
        s1 += q.w;
        s2 += q.w * q.w;
        const int64_t n0 = u0 + 128 * wa + r + 4 * h;
        if (t < p.Tv && n0 < p.N64) *reinterpret_cast<float4*>(srow + n0) = q;
      }
    }
    s1 += __shfl_xor(s1, 32);
    if (p.centred) {
      // sum (s - mean)^2 over these units, their mean from s1 (v41:1719-1721
      // over a 128-unit slice; the slices merge exactly in srw_tau_kernel)
      const int64_t nrow = p.N - (u0 + 128 * wa);
      const float n = static_cast<float>(nrow <= 0 ? 0 : (nrow < 128 ? nrow : 128));
      const float mu = n > 0.f ? s1 / n : 0.f;
      s2 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = 32 * i + 8 * (v >> 2) + (v & 3);
          const float d = r < nleft ? acc[i][j][v] - mu : 0.f;
          s2 += d * d;
        }
    }
    s2 += __shfl_xor(s2, 32);
    if (h == 0 && t < p.Tv) {
      float* m = p.mom + ((static_cast<int64_t>(2 * ct + wa)) * p.Tv + t) * 2;
      m[0] = s1;
      m[1] = s2;
    }
  }
}

// ---------------------------------------------------------------------------
// gate: XR of one tile, the v4.1 gate of the stored scores, P over S in place
// ---------------------------------------------------------------------------
struct FGateParams {
  const float* x;     // [T, D] (row v / routes)
  const float* read;  // [N, D]
  const float* tau;   // [Tv]
  float* P;           // [Tv, N64]: the scores in, P out (in place)
  float* tok_part;    // [2 CT][Tv][4]: sum gate, sum intensity, active count
  uint32_t* mask32;   // [Tv][mask_words32] or null
  float* G;           // [Tv, N] every unit's gate (SRW_FLAG_GATE_OUT) or null
  const float* sstd;  // [Tv] s_std (the v4.0.1 gate)
  int64_t mask_words32;
  int64_t Tv, N, N64, D;
  int routes, RT, CT;  // token tiles, unit tiles
  GateParams gp;
};

// tiles as f32_stats_kernel's.  GL: the v4.0.1 gate of _srw_inference
// (v401:1451-1453): z = (s - tau) / s_std, gate = z Phi(z) for z > 0; a unit
// is active where its gate is > 0, and the row sums carry z+ where v4.1 has
// the intensity
template <int MJ, bool GL>
__global__ __launch_bounds__(kFThreads, 1) void f32_gate_kernel(FGateParams p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wa = wave >> 1, wb = wave & 1, u = lane & 31, h = lane >> 5;
  int rt, ct;
  if (!ftile_of(p.RT, p.CT, rt, ct)) return;
  const int64_t u0 = static_cast<int64_t>(ct) * kFRows, v0 = static_cast<int64_t>(rt) * 64 * MJ;
  f32x16_t acc[4][MJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc[i][j] = f32x16_t{};
  {
    const FOpnd<8> A = make_fopnd<8>(p.read, p.D, u0, p.N, 1, wave, lane);
    const FOpnd<2 * MJ> B = make_fopnd<2 * MJ>(p.x, p.D, v0, p.Tv, p.routes, wave, lane);
    fgemm_loop(acc, A, B, 0, static_cast<int>(p.D / kFK), lds, 4 * wa, MJ * wb, wave, lane);
  }

  // gate epilogue (v41:1723-1735) in the reference's fp32 expression order;
  // four consecutive units per load / store
  const int64_t nleft = p.N - (u0 + 128 * wa + 4 * h);  // units of this wave-row left in the pool
  const float k_exp2 = -p.gp.sharp * 1.4426950408889634f;   // e^(-sharpness m) = 2^(m k_exp2)
#pragma unroll
  for (int j = 0; j < MJ; ++j) {
    const int64_t t = v0 + 32 * (MJ * wb + j) + u;
    const bool tok = t < p.Tv;
    float* prow = p.P + (tok ? t : p.Tv - 1) * p.N64;
    const float tau = p.tau[tok ? t : p.Tv - 1];
    const float sstd = GL ? p.sstd[tok ? t : p.Tv - 1] : 1.f;
    float gs = 0.f, is = 0.f;
    int na = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t m = 0;  // pass bits of the 32-unit block: element v at bit unit_of_acc(v, h)
#pragma unroll
      for (int v = 0; v < 16; v += 4) {
        const int r = 32 * i + 8 * (v >> 2);
        const int64_t nb = u0 + 128 * wa + r + 4 * h;
        const bool in_row = nb < p.N64;  // the last unit tile may reach past the row's N64 columns
        float4 q = in_row ? *reinterpret_cast<const float4*>(prow + nb) : float4{0.f, 0.f, 0.f, 0.f};
        float e[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          // margin = (s - tau) - thr, sigmoid(sharpness margin) through the
          // hardware exp2 (within 2 ulp of expf), intensity and gate in the
          // reference's order (v41:1723-1728)
          const bool ok = r + k < nleft;  // units past N count for nothing
          float gate;
          if constexpr (GL) {
            const GeluOut go = gate_gelu_v401(e[k], tau, sstd);
            gate = ok ? go.gate : 0.f;
            is += ok && go.z > 0.f ? go.z : 0.f;
            if (gate > 0.f) m |= 1u << (8 * (v >> 2) + 4 * h + k);
          } else {
            const float margin = (e[k] - tau) - p.gp.thr;
            const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(margin * k_exp2));
            const float inten = p.gp.eps + fminf(fmaxf(margin - p.gp.cut, 0.0f), p.gp.maxi);
            gate = ok ? act * inten : 0.f;
            is += ok ? inten : 0.f;
            if (ok && act > 0.5f) m |= 1u << (8 * (v >> 2) + 4 * h + k);
          }
          gs += gate;
          if (p.G && tok && ok) p.G[t * p.N + nb + k] = gate;
          e[k] = gate * acc[i][j][v + k];  // P = gate * xr (v41:1735)
        }
        if (tok && in_row) *reinterpret_cast<float4*>(prow + nb) = float4{e[0], e[1], e[2], e[3]};
      }
      na += __builtin_popcount(m);
      m |= __shfl_xor(m, 32);
      const int64_t word = (u0 + 128 * wa + 32 * i) / 32;
      if (p.mask32 && h == 0 && tok && word < p.mask_words32) p.mask32[t * p.mask_words32 + word] = m;
    }
    gs += __shfl_xor(gs, 32);
    is += __shfl_xor(is, 32);
    na += __shfl_xor(na, 32);
    if (h == 0 && tok) {
      float* tp = p.tok_part + (static_cast<int64_t>(2 * ct + wa) * p.Tv + t) * 4;
      tp[0] = gs;
      tp[1] = is;
      tp[2] = static_cast<float>(na);
      tp[3] = 0.f;
    }
  }
}

// ---------------------------------------------------------------------------
// write: OUT partial of one N-split = P[:, split units] . W^T[:, split units]^T
// ---------------------------------------------------------------------------
struct FWriteParams {
  const float* P;   // [Tv, N64]
  const float* wt;  // [D, N64]
  float* out_part;  // [S][Tv][D]
  int64_t Tv, N64, D;
  int S, RT, DT, nkb;  // RT, DT: token and column tiles of this kernel's tile shape; nkb: 32-unit k blocks
  int W8;              // (token tile, split) pairs per XCD
};

// A workgroup computes a (32 GA tokens) x (32 GB columns) tile of one split's
// partial; its waves hold MI x MJ MFMA tiles each, GB / MJ waves across the
// columns.  Shapes: 128 x 192 (GA = 4, GB = 6, 2 x 2 waves of 64 x 96: 80 KB
// of LDS and ~200 registers a wave, two workgroups per CU) where it pads no
// more output columns than 256 x 256 (GA = GB = 8, 2 x 2 waves of 128 x 128,
// one workgroup per CU), e.g. D = 384 (128 x 384 tiles, one workgroup per
// CU: 14% slower).
template <int GA, int GB, int MI, int MJ>
__global__ __launch_bounds__(kFThreads, 1) void f32_write_kernel(FWriteParams p) {
  static_assert(GA % MI == 0 && GB % MJ == 0 && (GA / MI) * (GB / MJ) == kFThreads / 64,
                "one accumulator block per wave");
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int WB = GB / MJ;
  const int wa = wave / WB, wb = wave % WB, u = lane & 31, h = lane >> 5;
  // XCD x (blockIdx % 8) takes the W8 consecutive (token tile, split) pairs
  // from x W8 on, token tile fastest, each with its DT column tiles in a row:
  // the column tiles share the P tile and the token tiles of a split share
  // its W^T rows in the XCD's L2.
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int dt = k % p.DT;
  const int w = x * p.W8 + k / p.DT;
  if (k / p.DT >= p.W8 || w >= p.RT * p.S) return;
  const int rt = w % p.RT, split = w / p.RT;
  const int64_t kb0 = static_cast<int64_t>(p.nkb) * split / p.S, kb1 = static_cast<int64_t>(p.nkb) * (split + 1) / p.S;
  const int64_t v0 = static_cast<int64_t>(rt) * 32 * GA, d0 = static_cast<int64_t>(dt) * 32 * GB;
  const FOpnd<GA> A = make_fopnd<GA>(p.P, p.N64, v0, p.Tv, 1, wave, lane);
  const FOpnd<GB> B = make_fopnd<GB>(p.wt, p.N64, d0, p.D, 1, wave, lane);
  f32x16_t acc[MI][MJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc[i][j] = f32x16_t{};
  fgemm_loop(acc, A, B, kb0 * kFK, static_cast<int>(kb1 - kb0), lds, MI * wa, MJ * wb, wave, lane);

  float* dst = p.out_part + static_cast<int64_t>(split) * p.Tv * p.D;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t t = v0 + 32 * (MI * wa + i) + 8 * (v >> 2) + 4 * h + (v & 3);
      if (t >= p.Tv) continue;
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        const int64_t d = d0 + 32 * (MJ * wb + j) + u;
        if (d < p.D) dst[t * p.D + d] = acc[i][j][v];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// final: per row the gate kernel's partials in tile order, den, and out =
// (sum over splits of the partial rows) / den * scale in fp32 (v41:1736-1737).
// One workgroup per row.
// ---------------------------------------------------------------------------
struct FFinalParams {
  const float* out_part;  // [S][Tv][D]
  const float* tok_part;  // [S_tok][Tv][4]
  float* out;             // [Tv, D]
  float* gate_sum;
  float* den;
  int32_t* n_active;
  int64_t Tv, D;
  int S, S_tok;
  int den_gate;           // den = max(sum gate, 1) (the v4.0.1 gate, v401:1461-1462)
  float scale;
};

__global__ __launch_bounds__(256) void f32_final_kernel(FFinalParams p) {
  __shared__ float red[3][4];
  __shared__ float den_s;
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float g = 0.f, in = 0.f, na = 0.f;
  for (int s = threadIdx.x; s < p.S_tok; s += 256) {
    const float4 q = *reinterpret_cast<const float4*>(p.tok_part + (static_cast<int64_t>(s) * p.Tv + t) * 4);
    g += q.x;
    in += q.y;
    na += q.z;
  }
  g = wave_sum(g);
  in = wave_sum(in);
  na = wave_sum(na);
  if (lane == 0) {
    red[0][wave] = g;
    red[1][wave] = in;
    red[2][wave] = na;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const float G = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    const float I = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    const float A = red[2][0] + red[2][1] + red[2][2] + red[2][3];
    const float den = fmaxf(p.den_gate ? G : I, 1.0f);  // v41:1736, v401:1461-1462
    den_s = den;
    if (p.gate_sum) p.gate_sum[t] = G;
    if (p.den) p.den[t] = den;
    if (p.n_active) p.n_active[t] = static_cast<int32_t>(A);
  }
  __syncthreads();
  const float den = den_s;
  for (int64_t d = threadIdx.x; d < p.D; d += 256) {
    float acc = 0.f;
    for (int s = 0; s < p.S; ++s) acc += p.out_part[(static_cast<int64_t>(s) * p.Tv + t) * p.D + d];
    p.out[t * p.D + d] = acc / den * p.scale;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct FGeo {
  int64_t Tv, N, N64;
  int CT, nkb;
  int RTq;                // score / gate kernels: 64-token tiles
  bool w192;              // write tiles of 128 tokens x 192 columns (else 256 x 256)
  int WRT, DT, S, W8;     // write: token tiles, column tiles, splits, pairs per XCD
};

int64_t fal256(int64_t b) { return (b + 255) & ~static_cast<int64_t>(255); }

FGeo fgeo(const srw_desc_t& d) {
  FGeo g{};
  g.Tv = d.T * d.n_routes;
  g.N = d.n_units;
  g.N64 = (g.N + kFNAlign - 1) / kFNAlign * kFNAlign;
  g.CT = static_cast<int>((g.N + kFRows - 1) / kFRows);
  g.nkb = static_cast<int>(g.N64 / kFK);
  g.RTq = static_cast<int>((g.Tv + 63) / 64);  // score and gate kernels: 256-unit x 64-token tiles
  // write tile shape: 192 wide unless that pads more output columns
  const int64_t D = d.d_model, pad256 = (D + 255) / 256 * 256 - D, pad192 = (D + 191) / 192 * 192 - D;
  g.w192 = pad192 <= pad256;
  const int wr = g.w192 ? 128 : 256, wc = g.w192 ? 192 : 256;
  g.WRT = static_cast<int>((g.Tv + wr - 1) / wr);
  g.DT = static_cast<int>((D + wc - 1) / wc);
  // splits of the write GEMM: enough workgroups for 256 CUs, each at least
  // four k blocks
  const int64_t per_split = static_cast<int64_t>(g.WRT) * g.DT;
  int64_t S = (512 + per_split - 1) / per_split;
  const int64_t most = g.nkb / 4 > 1 ? g.nkb / 4 : 1;
  S = S < 1 ? 1 : (S > most ? most : S);
  g.S = static_cast<int>(S);
  g.W8 = static_cast<int>((static_cast<int64_t>(g.WRT) * g.S + 7) / 8);
  return g;
}

struct FLayout {
  size_t wt, P, mom, tau, out_part, tok_part, rn, wn, sstd, total;
};

FLayout flayout(const srw_desc_t& d, const FGeo& g) {
  FLayout l{};
  size_t off = 0;
  l.wt = off;
  off += fal256(d.d_model * g.N64 * 4);
  l.P = off;
  off += fal256(g.Tv * g.N64 * 4);
  l.mom = off;
  off += fal256(static_cast<int64_t>(2 * g.CT) * g.Tv * 2 * 4);
  l.tau = off;
  off += fal256(g.Tv * 4);
  l.out_part = off;
  off += fal256(static_cast<int64_t>(g.S) * g.Tv * d.d_model * 4);
  l.tok_part = off;
  off += fal256(static_cast<int64_t>(2 * g.CT) * g.Tv * 4 * 4);
  // the v4.0.1 gate: forward-normalised R and W (v401:1456-1457), s_std per row
  l.rn = l.wn = l.sstd = off;
  if (d.gate == SRW_GATE_GELU_V401) {
    l.wn = l.rn + fal256(d.n_units * d.d_model * 4);
    l.sstd = l.wn + fal256(d.n_units * d.d_model * 4);
    off = l.sstd + fal256(g.Tv * 4);
  }
  l.total = off;
  return l;
}

}  // namespace

bool tiled_f32_supports(const srw_desc_t& d) {
  if (d.dtype != SRW_F32) return false;  // v4.1, or the v4.0.1 GELU gate of _srw_inference
  // operand offsets within a 256-row tile are 32-bit: 256 rows of the
  // [T, N64] fp32 scores / P must stay below 4 GiB
  if (256 * ((d.n_units + 63) / 64 * 64) * 4 >= (int64_t(1) << 32)) return false;
  if (d.stats_mode != SRW_STATS_ONEPASS && d.stats_mode != SRW_STATS_CENTERED) return false;
  if (d.flags & (SRW_FLAG_DIAG | SRW_FLAG_EMULATE | SRW_FLAG_NO_FAST)) return false;
  if (d.n_routes != 1 && d.n_routes != 2) return false;
  if (d.d_model % kFK != 0 || d.d_route % kFK != 0) return false;
  return true;
}

size_t tiled_f32_workspace_bytes(const srw_desc_t& d) { return flayout(d, fgeo(d)).total; }

hipError_t tiled_f32_forward(const LaunchArgs& a) {
  const srw_desc_t& d = a.d;
  const FGeo g = fgeo(d);
  const FLayout l = flayout(d, g);
  if (a.ws_bytes < l.total) return hipErrorInvalidValue;
  float* wt = reinterpret_cast<float*>(a.ws + l.wt);
  float* P = reinterpret_cast<float*>(a.ws + l.P);
  float* mom = reinterpret_cast<float*>(a.ws + l.mom);
  float* tau = reinterpret_cast<float*>(a.ws + l.tau);
  float* out_part = reinterpret_cast<float*>(a.ws + l.out_part);
  float* tok_part = reinterpret_cast<float*>(a.ws + l.tok_part);
  const int D = static_cast<int>(d.d_model);
  hipError_t e;
  static_assert(kFGemmLds <= 160 * 1024, "LDS per workgroup");
  const bool gl = d.gate == SRW_GATE_GELU_V401;
  for (const void* fn : {reinterpret_cast<const void*>(f32_stats_kernel<1>),
                         reinterpret_cast<const void*>(f32_gate_kernel<1, false>),
                         reinterpret_cast<const void*>(f32_gate_kernel<1, true>),
                         reinterpret_cast<const void*>(f32_write_kernel<8, 8, 4, 4>),
                         reinterpret_cast<const void*>(f32_write_kernel<4, 6, 2, 3>)})
    if ((e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kFGemmLds)) != hipSuccess) return e;

  // the v4.0.1 gate reads forward-normalised rows (kept in the workspace
  // across calls that declare the pool cached)
  const float* read_rows = static_cast<const float*>(a.in.read);
  const float* write_rows = static_cast<const float*>(a.in.write);
  if (gl) {
    float* rn = reinterpret_cast<float*>(a.ws + l.rn);
    float* wn = reinterpret_cast<float*>(a.ws + l.wn);
    if (!(d.flags & SRW_FLAG_POOL_CACHED)) {
      if ((e = normalize_rows_f32(read_rows, rn, g.N, D, a.stream)) != hipSuccess) return e;
      if ((e = normalize_rows_f32(write_rows, wn, g.N, D, a.stream)) != hipSuccess) return e;
    }
    read_rows = rn;
    write_rows = wn;
  }
  if (!(d.flags & SRW_FLAG_POOL_CACHED)) {
    const dim3 grid_p(static_cast<unsigned>(g.N64 / 64), static_cast<unsigned>((D + 63) / 64));
    hipLaunchKernelGGL(pack_wt_f32_kernel, grid_p, dim3(256), 0, a.stream, write_rows, wt, g.N, g.N64, D);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // score and gate kernels: 256-unit x 64-token tiles, two stages of 256 + 64 operand rows
  const dim3 grid_q(static_cast<unsigned>(8 * g.RTq * ((g.CT + 7) / 8)));
  constexpr size_t kLdsQ = 2 * (8 + 2) * kFGroupBytes;
  FStatsParams sp{};
  sp.h = static_cast<const float*>(a.in.h);
  sp.emb = static_cast<const float*>(a.in.emb);
  sp.S = P;
  sp.mom = mom;
  sp.Tv = g.Tv;
  sp.N = g.N;
  sp.N64 = g.N64;
  sp.dr = d.d_route;
  sp.centred = d.stats_mode == SRW_STATS_CENTERED;
  sp.RT = g.RTq;
  sp.CT = g.CT;
  hipLaunchKernelGGL(f32_stats_kernel<1>, grid_q, dim3(kFThreads), kLdsQ, a.stream, sp);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  // tau per row from the 2 CT partials of 128 units (centred: merged by
  // Chan's formula, no second pass over the stored scores)
  float* sstd = gl ? reinterpret_cast<float*>(a.ws + l.sstd) : nullptr;
  if ((e = launch_tau(mom, a.in.tau_offset, tau, g.Tv, 2 * g.CT, g.N, 2, nullptr,
                      d.stats_mode == SRW_STATS_CENTERED ? kTauChan : kTauOnePass, a.stream, sstd, 128)) !=
      hipSuccess)
    return e;

  FGateParams gp{};
  gp.x = static_cast<const float*>(a.in.x);
  gp.read = read_rows;
  gp.sstd = sstd;
  gp.tau = tau;
  gp.P = P;
  gp.tok_part = tok_part;
  gp.mask32 = reinterpret_cast<uint32_t*>(a.o.pass_mask);
  gp.G = (d.flags & SRW_FLAG_GATE_OUT) ? a.o.gate : nullptr;
  gp.mask_words32 = 2 * a.words;
  gp.Tv = g.Tv;
  gp.N = g.N;
  gp.N64 = g.N64;
  gp.D = D;
  gp.routes = d.n_routes;
  gp.gp = a.gp;
  dominant_kernel_begin(a.stream);
  gp.RT = g.RTq;
  gp.CT = g.CT;
  if (gl)
    hipLaunchKernelGGL((f32_gate_kernel<1, true>), grid_q, dim3(kFThreads), kLdsQ, a.stream, gp);
  else
    hipLaunchKernelGGL((f32_gate_kernel<1, false>), grid_q, dim3(kFThreads), kLdsQ, a.stream, gp);
  dominant_kernel_end(a.stream);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  FWriteParams wp{};
  wp.P = P;
  wp.wt = wt;
  wp.out_part = out_part;
  wp.Tv = g.Tv;
  wp.N64 = g.N64;
  wp.D = D;
  wp.S = g.S;
  wp.RT = g.WRT;
  wp.DT = g.DT;
  wp.nkb = g.nkb;
  wp.W8 = g.W8;
  const unsigned grid_w = static_cast<unsigned>(8 * g.DT * g.W8);
  if (g.w192)
    hipLaunchKernelGGL((f32_write_kernel<4, 6, 2, 3>), dim3(grid_w), dim3(kFThreads), 2 * (4 + 6) * kFGroupBytes,
                       a.stream, wp);
  else
    hipLaunchKernelGGL((f32_write_kernel<8, 8, 4, 4>), dim3(grid_w), dim3(kFThreads), kFGemmLds, a.stream, wp);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  FFinalParams fp{};
  fp.out_part = out_part;
  fp.tok_part = tok_part;
  fp.out = static_cast<float*>(a.o.out);
  fp.gate_sum = a.o.gate_sum;
  fp.den = a.o.den;
  fp.n_active = a.o.n_active;
  fp.Tv = g.Tv;
  fp.D = D;
  fp.S = g.S;
  fp.S_tok = 2 * g.CT;
  fp.den_gate = gl;
  fp.scale = d.scale;
  hipLaunchKernelGGL(f32_final_kernel, dim3(static_cast<unsigned>(g.Tv)), dim3(256), 0, a.stream, fp);
  return hipGetLastError();
}

}  // namespace srw

// srw_mfma.hip -- bf16 matrix-core SRW forward for gfx950.
//
// Replaces the two chunk scans of fused_gate_srw (models/dawn_spatial_v41_exp.py
// :433-577) with four kernels on the caller's stream:
//
//   pack      W [N, D] -> W^T fragments: the write GEMM contracts over units,
//             which are the strided axis of W, so W is re-laid once per call in
//             the order the matrix core's B operand wants (unit-contiguous, in
//             the unit permutation the gate registers come out in).
//   stats     S = H.E^T on the matrix cores, rounded to bf16 (v41:439), and the
//             per-token power sums sum s, sum s^2 per N-split (v41:441-442).
//   main      per (token tile, N-split): tau from the moments (v41:461-464),
//             then for every 32-unit tile: S^T = E_t.H^T and XR^T = R_t.X^T
//             (MFMA), the v4.1 gate in registers (v41:506-511), P = bf16(bf16(g)
//             * bf16(xr)) (v41:516-518) fed straight back as the A operand of
//             OUT += P.W_t (MFMA) -- the [T, N] gate never leaves the registers.
//             Emits fp32 partial OUT, per-token partial sum gate / sum
//             intensity / active count, and the pass bitmask.
//   finalize  sums the N-split partials, rounds each reference chunk's write
//             GEMM to bf16 (v41:518, chunk plan v41:416-420), den =
//             max(sum intensity, 1), out = bf16(raw / den) (v41:584-586).
//
// Matrix-core layout facts used throughout (v_mfma_f32_32x32x16_bf16, wave64):
//   A operand: lane l holds A[l % 32][8 (l / 32) + i], i = 0..7
//   B operand: lane l holds B[8 (l / 32) + i][l % 32]
//   C/D:       acc[v] of lane l is C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32]
// so the gate values a lane holds after the score GEMM (one token, 16 units)
// are already an A operand of the write GEMM, under the unit permutation
// unit_of_k() below; the packed W^T uses the same permutation.
//
// Workgroup: 4 waves, 32 tokens per wave (token tile 128); X (and H) live in
// VGPRs for the whole kernel, the fp32 OUT tile [32 x D] per wave in the
// accumulator registers.  E, R and W^T tiles stream through LDS in a double
// buffer filled by direct global->LDS loads, laid out fragment-major so every
// LDS read is one conflict-free 16-byte row per lane.

#include <type_traits>

#include "srw_internal.hpp"
#include "srw_mfma_util.hpp"

namespace srw {

namespace {

constexpr int kThreads = 256;     // 4 waves
constexpr int kTokTile = 128;     // tokens per workgroup
constexpr int kUnitTile = 32;     // units per tile
constexpr int kTargetBlocks = 256;

// Lane exchanges within 32-lane halves, on the vector ALU (DPP and the gfx950
// row swap) rather than the LDS crossbar: the value of lane (lane ^ m).
__device__ inline float as_f(int v) { return __builtin_bit_cast(float, v); }
__device__ inline int as_i(float v) { return __builtin_bit_cast(int, v); }
template <int M>
__device__ inline float lane_xor(float v, int lane) {
  if constexpr (M == 1) return as_f(__builtin_amdgcn_mov_dpp(as_i(v), 0xB1, 0xF, 0xF, true));  // quad_perm [1,0,3,2]
  if constexpr (M == 2) return as_f(__builtin_amdgcn_mov_dpp(as_i(v), 0x4E, 0xF, 0xF, true));  // quad_perm [2,3,0,1]
  if constexpr (M == 4) {
    const float up = as_f(__builtin_amdgcn_mov_dpp(as_i(v), 0x104, 0xF, 0xF, true));  // row_shl:4
    const float dn = as_f(__builtin_amdgcn_mov_dpp(as_i(v), 0x114, 0xF, 0xF, true));  // row_shr:4
    return (lane & 4) ? dn : up;
  }
  if constexpr (M == 8) return as_f(__builtin_amdgcn_mov_dpp(as_i(v), 0x128, 0xF, 0xF, true));  // row_ror:8
  if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(as_i(v), as_i(v), false, false);
    return as_f((lane & 16) ? r[0] : r[1]);
  }
}

// Reduce-scatter of 16 values per lane over the 32 lanes of each half: on
// return a[0] of lane l holds the reduction, over the half's 32 lanes, of
// element k = 8 (l & 1) + 4 (l >> 1 & 1) + 2 (l >> 2 & 1) + (l >> 3 & 1).
template <class Op>
__device__ inline void reduce_scatter16(float (&a)[16], int lane, Op op) {
  auto step = [&](auto mtag, int cnt) {
    constexpr int M = decltype(mtag)::value;
    const bool up = lane & M;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k >= cnt / 2) break;
      const float send = up ? a[k] : a[k + cnt / 2], keep = up ? a[k + cnt / 2] : a[k];
      a[k] = op(keep, lane_xor<M>(send, lane));
    }
  };
  step(std::integral_constant<int, 1>{}, 16);
  step(std::integral_constant<int, 2>{}, 8);
  step(std::integral_constant<int, 4>{}, 4);
  step(std::integral_constant<int, 8>{}, 2);
  a[0] = op(a[0], lane_xor<16>(a[0], lane));
}


// A 32-row tile of a row-major bf16 [rows, K] array (E or R), staged in LDS
// as K / 16 one-KB blocks.  Load block j moves whole 128-byte lines (8 rows x
// 128 B; 16 rows x 64 B when K = 32): a wave load that touches 32 B of each of
// 32 rows costs the texture path four times the line requests and halves the
// global->LDS rate.  The 16-byte pieces of each row are XOR-swizzled by row,
// so that the MFMA fragment reads (32 rows x 32 B) are free of bank conflicts:
// the LDS serves a ds_read_b128 16 lanes (256 B) at a time, and each group of
// 16 lanes hits 16 distinct 16-byte slots.
template <int KF>  // K / 16: MFMA k-steps per row
struct RowTile {
  static constexpr int K = KF * 16;
  static constexpr int PPR = KF * 2 < 8 ? KF * 2 : 8;  // 16-B pieces of a row per block
  static constexpr int RPI = 64 / PPR;                 // rows per block
  static constexpr int RG = 32 / RPI;                  // row groups
  static constexpr int NM = PPR / 2;                   // k-steps per block row
  __host__ __device__ static constexpr int swz(int r) {
    return PPR == 8 ? (r % 8) ^ ((r / 8) & 1) : (r / 4) % 4;
  }
  // Byte offset, within block j's rows, of the 16 B `lane` loads: swz depends
  // on the row group of block j only through its parity (PPR = 8), so each
  // lane keeps two offsets; block j adds the wave-uniform block_off(j).
  __device__ static uint32_t lane_src(int lane, int parity) {
    const int r = lane / PPR;
    const int sw = PPR == 8 ? swz(r) ^ parity : swz(r);
    return static_cast<uint32_t>((r * K + 8 * ((lane % PPR) ^ sw)) * 2);
  }
  static constexpr int block_off(int j) { return (RPI * (j % RG) * K + 8 * (j / RG) * PPR) * 2; }
  // load block j of the tile whose first row is row0 (rows past `rows` read the last one);
  // lsrc = {lane_src(lane, 0), lane_src(lane, 1)}.  Whole tiles use a
  // wave-uniform base plus the lane offset.
  __device__ static void load(const uint16_t* a, int64_t row0, int64_t rows, int j, int lane, const uint32_t* lsrc,
                              char* tile) {
    if (row0 + 32 <= rows) {
      g2lds16(reinterpret_cast<const char*>(a) + (row0 * K * 2 + block_off(j)) + lsrc[(j % RG) & 1],
              tile + j * kFragBytes);
    } else {
      const int r = RPI * (j % RG) + lane / PPR;
      const int c = 8 * ((j / RG) * PPR + ((lane % PPR) ^ swz(r)));
      const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
      g2lds16(a + row * K + c, tile + j * kFragBytes);
    }
  }
  // LDS byte offset of the 16 B that `lane` feeds to MFMA k-step ks:
  // lane_off(lane, ks % NM) + step_off(ks)
  __device__ static int lane_off(int lane, int m) {
    const int u = lane & 31, h = lane >> 5;
    return (u / RPI) * kFragBytes + (PPR * (u % RPI) + ((2 * m + h) ^ swz(u))) * 16;
  }
  static constexpr int step_off(int ks) { return (ks / NM) * RG * kFragBytes; }
};


// The gate epilogue of a tile as 48 micro-steps (type * 16 + element):
// type 0 = bf16 score, margin, exp; 1 = sigmoid, intensity, gate; 2 = sums,
// pass bit, bf16 product.  Element v's three steps are spread two entries
// apart so each result has an MFMA's duration to land before it is used.
__device__ constexpr uint8_t kEpiStep[48] = {
    0, 1, 16, 2, 17, 32, 3, 18, 33, 4, 19, 34, 5, 20, 35, 6, 21, 36, 7, 22, 37, 8, 23, 38,
    9, 24, 39, 10, 25, 40, 11, 26, 41, 12, 27, 42, 13, 28, 43, 14, 29, 44, 15, 30, 45, 31, 46, 47};

struct Geometry {
  int64_t T, N, cs;      // tokens, units, reference chunk size (N if unchunked)
  int nc;                // reference chunks
  int spc;               // N-splits per chunk of the main kernel
  int S;                 // N-splits in total (nc * spc)
  int spc_st, S_st;      // the same for the moments kernel
  int TT;                // token tiles of the main kernel
  int TT_st;             // token tiles of the moments kernel
  int ntiles;            // ceil(N / 32): global 32-unit tiles
};

// Tile range [ta, tb) and unit bounds [lo, hi) of N-split `split`.  Splits
// never cross a reference chunk; tiles are globally 32-aligned, so a tile
// that holds a chunk boundary is shared by two splits (each masks the other's
// units).
__host__ __device__ inline void split_range(const Geometry& g, int spc, int split, int& ta, int& tb, int64_t& lo,
                                   int64_t& hi) {
  const int c = split / spc, sub = split % spc;
  const int64_t c_lo = c * g.cs;
  const int64_t c_hi = (c + 1) * g.cs < g.N ? (c + 1) * g.cs : g.N;
  const int t_lo = static_cast<int>(c_lo / kUnitTile);
  const int t_hi = static_cast<int>((c_hi + kUnitTile - 1) / kUnitTile);
  const int64_t nt = t_hi - t_lo;
  ta = t_lo + static_cast<int>(nt * sub / spc);
  tb = t_lo + static_cast<int>(nt * (sub + 1) / spc);
  lo = static_cast<int64_t>(ta) * kUnitTile > c_lo ? static_cast<int64_t>(ta) * kUnitTile : c_lo;
  hi = static_cast<int64_t>(tb) * kUnitTile < c_hi ? static_cast<int64_t>(tb) * kUnitTile : c_hi;
}

// Several independent calls in one launch per stage (srw_forward_batch): the
// parameters of each and the first block of each in the launch's grid.
constexpr int kMaxBatch = 4;
template <class P>
struct Batch {
  P p[kMaxBatch];
  int start[kMaxBatch + 1];  // call i owns blocks [start[i], start[i + 1])
  int n;
};
__device__ inline int batch_index(const int* start, int n, int bid) {
  int i = 0;
  for (int k = 1; k < n; ++k) i += bid >= start[k] ? 1 : 0;
  return i;
}

// ---------------------------------------------------------------------------
// pack: Wp[tile][db][j][lane][i] = W[32 tile + unit_of_k(j, lane/32, i)][32 db + lane%32]
// (zero beyond N).  One thread per 16-byte output fragment row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_w_kernel(const uint16_t* __restrict__ W, uint16_t* __restrict__ Wp,
                                                     int64_t N, int D, int64_t n_rows) {
  const int DB = D / 32;
  for (int64_t r = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; r < n_rows;
       r += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int lane = static_cast<int>(r & 63);
    const int64_t frag = r >> 6;                 // tile * (2 DB) + db * 2 + j
    const int j = static_cast<int>(frag & 1);
    const int db = static_cast<int>((frag >> 1) % DB);
    const int64_t tile = (frag >> 1) / DB;
    const int d = 32 * db + (lane & 31);
    const int half = lane >> 5;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t pair = 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int64_t u = tile * kUnitTile + unit_of_k(j, half, 2 * q + e);
        const uint32_t b = u < N ? W[u * D + d] : 0u;
        pair |= b << (16 * e);
      }
      w[q] = pair;
    }
    *reinterpret_cast<u32x4_t*>(Wp + r * 8) = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

// ---------------------------------------------------------------------------
// stats: per (token tile, split) the bf16-score power sums sum s, sum s^2.
// ---------------------------------------------------------------------------
struct StatsParams {
  const uint16_t* h;   // [T, dr]
  const uint16_t* emb; // [N, dr]
  float* mom;          // [S][T][2, 3 or 4]
  uint32_t* mask32;    // pass bitmask as uint32 words [T][mask_words32] (may be null)
  int64_t mask_words32;
  Geometry g;
  uint16_t* s_out;     // bf16 score buffer (score_tile_off layout) or null: plain moments only
  int64_t s_ld;        // kStatsRows / kStatsRowsOnly: row stride (elements) of the row-major s_out
};

// The bf16 scores as the scores-streaming main kernel reads them: per (token
// tile of 128 rows, 32-unit tile, 32-row token block) the 32 x 32 score
// accumulator of the wave that computed it, two 1 KB pieces of 64 lanes x
// 16 B (lane l's elements 0-7, then 8-15, in accumulator order: unit
// unit_of_acc(v, l / 32) of token l % 32).  Byte offset of a block:
constexpr int kScoreTileBytes = 4 * 2 * kFragBytes;  // one (token tile, unit tile)
__host__ __device__ inline int64_t score_tile_off(int ntiles, int64_t ttile, int64_t utile, int blk) {
  return (ttile * ntiles + utile) * kScoreTileBytes + static_cast<int64_t>(blk) * 2 * kFragBytes;
}

// MODE kStatsPlain: sum s, sum s^2 (v41:441-442); kStatsDiag: also sum s^3,
// s^4 (training diagnostics, v41:442-444; mom stride 4); kStatsChan: sum s,
// the sum of squares about the split's own mean and the split's unit count
// (mom stride 3), for _srw_inference's centred std (v41:1719-1721) in one
// pass: each tile's sum and sum of squares about the tile mean join the
// running (count, mean, M2) by Chan et al.'s pairwise update, and
// srw_tau_kernel merges the splits the same way.  kStatsRows: the plain
// moments, with the bf16 scores stored row-major ([T, s_ld], units as
// columns) instead of in the streaming layout; kStatsRowsOnly: the row-major
// store alone, no moments (the same tile loop as a plain bf16 GEMM with a
// bf16 output, K = 16 KH).
constexpr int kStatsPlain = 0, kStatsDiag = 1, kStatsChan = 3, kStatsRows = 4, kStatsRowsOnly = 5;
// A lane's running moments of one row's scores over the tiles of an N-split
// (the moments kernel, and the one-launch decode kernel, which runs the same
// arithmetic so that both give the same bits).  kStatsPlain / kStatsDiag:
// s1..s4 = sum s^k of the lane's elements; kStatsChan: cn, cmean = the
// split's unit count and mean so far, s1 = sum s, s2 = the centred sum of
// squares (both lane halves).
struct MomState {
  float s1, s2, s3, s4, cn, cmean;
};

// Join one 32-unit tile (sp: the lane's 16 packed bf16 scores, v41:503, in
// accumulator order) to the state; units outside [lo, hi) enter as zeros.
// FULL: the caller has checked that every unit of the tile is in [lo, hi).
template <int MODE, bool FULL = false>
__device__ __attribute__((always_inline)) inline void moment_tile(MomState& m, const uint32_t (&sp)[8], int64_t u0,
                                                                   int64_t lo, int64_t hi, int half) {
  const bool full = FULL || (u0 >= lo && u0 + kUnitTile <= hi);
  if constexpr (MODE == kStatsChan) {
    // this tile's units in the split, their sum and sum of squares about
    // their mean (both lane halves), joined to the running (count, mean, M2)
    const int64_t c_lo = u0 > lo ? u0 : lo, c_hi = u0 + kUnitTile < hi ? u0 + kUnitTile : hi;
    const float nt = static_cast<float>(c_hi > c_lo ? c_hi - c_lo : 0);
    float xs[16];
    bool oks[16];
    float ts = 0.f;
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      bool ok0 = true, ok1 = true;
      if (!full) {
        const int64_t ua = u0 + unit_of_acc(v, half), ub = u0 + unit_of_acc(v + 1, half);
        ok0 = ua >= lo && ua < hi;
        ok1 = ub >= lo && ub < hi;
      }
      xs[v] = ok0 ? lo_f32(sp[v >> 1]) : 0.f;
      xs[v + 1] = ok1 ? hi_f32(sp[v >> 1]) : 0.f;
      oks[v] = ok0;
      oks[v + 1] = ok1;
      ts += xs[v];
      ts += xs[v + 1];
    }
    ts += __shfl_xor(ts, 32);
    if (nt > 0.f) {
      const float mt = ts / nt;
      float m2 = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float dv = oks[v] ? xs[v] - mt : 0.f;
        m2 += __fmul_rn(dv, dv);
      }
      m2 += __shfl_xor(m2, 32);
      const float nn = m.cn + nt, dl = mt - m.cmean;
      m.cmean += dl * (nt / nn);
      m.s2 += m2 + dl * dl * (m.cn * nt / nn);
      m.s1 += ts;
      m.cn = nn;
    }
  } else {
    // sum s and sum s^2 of a packed bf16 pair in one v_dot2c_f32_bf16 each
    // (the squares of bf16 values are exact in fp32)
    const bf16x2_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      uint32_t q = sp[v >> 1];
      if (!full) {
        const int64_t ua = u0 + unit_of_acc(v, half), ub = u0 + unit_of_acc(v + 1, half);
        const bool ok0 = ua >= lo && ua < hi, ok1 = ub >= lo && ub < hi;
        q &= (ok0 ? 0x0000ffffu : 0u) | (ok1 ? 0xffff0000u : 0u);
      }
      const bf16x2_t sb = __builtin_bit_cast(bf16x2_t, q);
      m.s1 = __builtin_amdgcn_fdot2_f32_bf16(sb, ones, m.s1, false);
      m.s2 = __builtin_amdgcn_fdot2_f32_bf16(sb, sb, m.s2, false);
      if constexpr (MODE == kStatsDiag) {
        const float x0 = lo_f32(q), x1 = hi_f32(q);
        const float q0 = __fmul_rn(x0, x0), q1 = __fmul_rn(x1, x1);
        m.s3 += __fmul_rn(q0, x0);
        m.s4 += __fmul_rn(q0, q0);
        m.s3 += __fmul_rn(q1, x1);
        m.s4 += __fmul_rn(q1, q1);
      }
    }
  }
}

// The split's partial of row t: mom[split][t][MS] = (sum s, sum s^2 [, sum
// s^3, sum s^4]) or, kStatsChan, (sum s, M2, count); lane halves joined.
template <int MODE>
__device__ __attribute__((always_inline)) inline void moment_store(MomState m, float* mom, int split, int64_t T,
                                                                    int64_t t, int half) {
  constexpr int MS = MODE == kStatsDiag ? 4 : (MODE == kStatsChan ? 3 : 2);
  if constexpr (MODE != kStatsChan) {  // (the Chan sums already hold both lane halves)
    m.s1 += __shfl_xor(m.s1, 32);
    m.s2 += __shfl_xor(m.s2, 32);
  }
  if constexpr (MODE == kStatsDiag) {
    m.s3 += __shfl_xor(m.s3, 32);
    m.s4 += __shfl_xor(m.s4, 32);
  }
  if (half == 0 && t < T) {
    float* q = mom + (static_cast<int64_t>(split) * T + t) * MS;
    q[0] = m.s1;
    q[1] = m.s2;
    if constexpr (MODE == kStatsDiag) {
      q[2] = m.s3;
      q[3] = m.s4;
    }
    if constexpr (MODE == kStatsChan) q[2] = m.cn;
  }
}

// TBW 32-token blocks per wave (128 TBW tokens per workgroup): each E
// fragment read from LDS feeds TBW MFMAs, and a CU's E stream serves
// 128 TBW tokens.
template <int KH, int MODE, int TBW>
__device__ __attribute__((always_inline)) inline void stats_body(const StatsParams& p, const int bid) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  constexpr int STAGE = KH * kFragBytes;
  constexpr int DR = KH * 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int split = bid % p.g.S_st;
  const int ttile = bid / p.g.S_st;
  int64_t tt[TBW], tl[TBW];
#pragma unroll
  for (int b = 0; b < TBW; ++b) {
    tt[b] = static_cast<int64_t>(ttile) * kTokTile * TBW + 32 * (TBW * wave + b) + col;
    tl[b] = tt[b] < p.g.T ? tt[b] : p.g.T - 1;
  }
  int ta, tb;
  int64_t lo, hi;
  split_range(p.g, p.g.spc_st, split, ta, tb, lo, hi);

  // Zero the mask words that two splits share (chunk boundaries inside a
  // tile) and the unused upper half of the last 64-bit word; the main kernel
  // ORs into the former and never writes the latter.
  if (p.mask32 && split == 0) {
#pragma unroll
    for (int b = 0; b < TBW; ++b) {
      const int64_t t = tt[b];
      for (int c = 1; c < p.g.nc; ++c) {
        const int64_t bd = c * p.g.cs;
        if (bd % kUnitTile && half == 0 && t < p.g.T) p.mask32[t * p.mask_words32 + bd / kUnitTile] = 0u;
      }
      if ((p.g.ntiles & 1) && half == 0 && t < p.g.T) p.mask32[t * p.mask_words32 + p.g.ntiles] = 0u;
    }
  }

  u32x4_t hq[TBW][KH];
#pragma unroll
  for (int b = 0; b < TBW; ++b) {
#pragma unroll
    for (int ks = 0; ks < KH; ++ks)
      hq[b][ks] = *reinterpret_cast<const u32x4_t*>(p.h + tl[b] * DR + 16 * ks + 8 * half);
  }

  using TileE = RowTile<KH>;
  const uint32_t lsrc[2] = {TileE::lane_src(lane, 0), TileE::lane_src(lane, 1)};
  auto issue = [&](int tile, int stage) {
    for (int j = wave; j < KH; j += 4)
      TileE::load(p.emb, static_cast<int64_t>(tile) * kUnitTile, p.g.N, j, lane, lsrc, lds + stage * STAGE);
  };
  int le[TileE::NM];
#pragma unroll
  for (int m = 0; m < TileE::NM; ++m) le[m] = TileE::lane_off(lane, m);

  MomState ms[TBW];
#pragma unroll
  for (int b = 0; b < TBW; ++b) ms[b] = MomState{};
  // score store (plain moments, one block per wave): each tile's packed
  // scores go out at the start of the next tile's MFMAs, so the stores have
  // a whole tile to complete before the end-of-tile vmcnt wait.  A tile that
  // two splits share (a chunk boundary inside it) is stored by the split
  // holding its first unit.
  constexpr bool ROWS = MODE == kStatsRows || MODE == kStatsRowsOnly;
  constexpr bool STORE = TBW == 1 && (MODE == kStatsPlain || MODE == kStatsDiag || MODE == kStatsChan || ROWS);
  uint32_t spd[8];
  char* sdst = nullptr;
  // Non-temporal stores (and loads in the main kernel): 206 MB per Know-pool
  // call at T = 4096 that would otherwise displace the pool tiles the other
  // token tiles share, in L2 and in the last-level cache across kernels
  // (measured: moments kernel 101 -> 87 us, pack 12.8 -> 9.1 us).
  auto store_scores = [&]() {
    if constexpr (ROWS) {
      // row-major: units 16 half .. 16 half + 15 of the lane's row (the
      // words as rows_words left them), two 16-byte stores
      *reinterpret_cast<u32x4_t*>(sdst) = u32x4_t{spd[0], spd[1], spd[4], spd[5]};
      *reinterpret_cast<u32x4_t*>(sdst + 16) = u32x4_t{spd[2], spd[3], spd[6], spd[7]};
    } else {
      __builtin_nontemporal_store(u32x4_t{spd[0], spd[1], spd[2], spd[3]}, reinterpret_cast<u32x4_t*>(sdst));
      __builtin_nontemporal_store(u32x4_t{spd[4], spd[5], spd[6], spd[7]},
                                  reinterpret_cast<u32x4_t*>(sdst + kFragBytes));
    }
  };
  if (ta < tb) {
    issue(ta, 0);
    wait_vm0();
    __syncthreads();
  }
  for (int tile = ta; tile < tb; ++tile) {
    const int st = (tile - ta) & 1;
    const bool pre = tile + 1 < tb;  // the next tile's loads go out between this one's MFMAs
    f32x16_t acc[TBW];
#pragma unroll
    for (int b = 0; b < TBW; ++b) acc[b] = f32x16_t{};
    const char* base = lds + st * STAGE;
    auto frag = [&](int ks) {
      return *reinterpret_cast<const u32x4_t*>(base + le[ks % TileE::NM] + TileE::step_off(ks));
    };
    // the next tile's blocks (this wave's share: blocks wave, wave + 4, ...),
    // requested before this tile's k-loop; a whole tile inside the pool from
    // a uniform base plus the lane's offset
    if (pre) {
      const int64_t row0 = static_cast<int64_t>(tile + 1) * kUnitTile;
      if (row0 + kUnitTile <= p.g.N) {
        const char* enext = reinterpret_cast<const char*>(p.emb) + row0 * TileE::K * 2;
#pragma unroll
        for (int j0 = 0; j0 < KH; j0 += 4) {
          const int j = j0 + wave;
          if (KH % 4 == 0 || j < KH)
            g2lds16(enext + TileE::block_off(j) + lsrc[(j % TileE::RG) & 1], lds + (st ^ 1) * STAGE + j * kFragBytes);
        }
      } else {
        for (int j = wave; j < KH; j += 4) TileE::load(p.emb, row0, p.g.N, j, lane, lsrc, lds + (st ^ 1) * STAGE);
      }
    }
    constexpr int PF = 4;
    u32x4_t ef[PF];
#pragma unroll
    for (int g = 0; g < PF; ++g)
      if (g < KH) ef[g] = frag(g);
#pragma unroll
    for (int ks = 0; ks < KH; ++ks) {
      if constexpr (STORE) {
        if (ks == 0 && sdst) {
          store_scores();
          sdst = nullptr;
        }
      }
      const u32x4_t e = ef[ks % PF];
      if (ks + PF < KH) ef[ks % PF] = frag(ks + PF);
#pragma unroll
      for (int b = 0; b < TBW; ++b) acc[b] = mfma(e, hq[b][ks], acc[b]);
      __builtin_amdgcn_sched_barrier(0);
    }
    const int64_t u0 = static_cast<int64_t>(tile) * kUnitTile;
    if constexpr (STORE) {
      // the bf16 scores (v41:503), packed whether or not this split stores
      // them: a conditional assignment would keep the previous tile's words
      // alive in copies
#pragma unroll
      for (int v = 0; v < 16; v += 2) spd[v >> 1] = pack_bf16(acc[0][v], acc[0][v + 1]);
      if constexpr (ROWS) {
        // word k of lane (row, half) holds units 8 (k / 2) + 4 half + 2 (k %
        // 2) + {0, 1} of the tile.  Swapping words k and 4 + k between the
        // two lanes of a row (v_permlane32_swap: the upper half of the first
        // operand with the lower half of the second) leaves lane half with
        // units 16 half .. 16 half + 15 as words 0, 1, 4, 5, 2, 3, 6, 7.
        // Every lane of the wave runs it (the stores below are per lane).
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const auto r = __builtin_amdgcn_permlane32_swap(spd[k], spd[4 + k], false, false);
          spd[k] = r[0];
          spd[4 + k] = r[1];
        }
        if (u0 >= lo && tt[0] < p.g.T)
          sdst = reinterpret_cast<char*>(p.s_out) + (tt[0] * p.s_ld + u0 + 16 * half) * 2;
      } else {
        if (p.s_out && u0 >= lo)
          sdst = reinterpret_cast<char*>(p.s_out) + score_tile_off(p.g.ntiles, ttile, tile, wave) + lane * 16;
      }
    }
    // this tile's moments (v41:441-444): the packed bf16 scores (v41:503),
    // units outside the split excluded
    if constexpr (MODE != kStatsRowsOnly) {
      // a uniform branch between the whole tiles (all but a split's edge
      // tiles) and the masked ones: as selects, the masking's 64-bit unit
      // compares ran on every tile (~4.6 VALU instructions per MFMA)
      const bool full = u0 >= lo && u0 + kUnitTile <= hi;
#pragma unroll
      for (int b = 0; b < TBW; ++b) {
        uint32_t sp[8];
#pragma unroll
        for (int v = 0; v < 16; v += 2) sp[v >> 1] = pack_bf16(acc[b][v], acc[b][v + 1]);
        if (full)
          moment_tile<MODE, true>(ms[b], sp, u0, lo, hi, half);
        else
          moment_tile<MODE, false>(ms[b], sp, u0, lo, hi, half);
      }
    }
    wait_vm0();
    __syncthreads();
  }
  if constexpr (STORE) {
    if (sdst) store_scores();
  }
  if constexpr (MODE != kStatsRowsOnly) {
#pragma unroll
    for (int b = 0; b < TBW; ++b) moment_store<MODE>(ms[b], p.mom, split, p.g.T, tt[b], half);
  }
}

// Three workgroups per CU where the registers allow it without spills (not
// with the diagnostics' extra power sums, nor in the batch kernel): a third
// wave per SIMD covers the tile loop's LDS and barrier waits (measured 97.1
// -> 93.6 us at the Know pool).
template <int MODE>
constexpr int stats_min_blocks() { return MODE == kStatsDiag ? 2 : 3; }
template <int KH, int MODE, int TBW>
__global__ __launch_bounds__(kThreads, stats_min_blocks<MODE>()) void srw_stats_kernel(StatsParams p) {
  stats_body<KH, MODE, TBW>(p, blockIdx.x);
}
template <int KH, int MODE>
__global__ __launch_bounds__(kThreads) void srw_stats_batch_kernel(Batch<StatsParams> b) {  // (3 would spill)
  const int i = batch_index(b.start, b.n, blockIdx.x);
  stats_body<KH, MODE, 1>(b.p[i], blockIdx.x - b.start[i]);
}

// ---------------------------------------------------------------------------
// main: fused score / read / gate / write for one (token tile, N-split).
// ---------------------------------------------------------------------------
// Per-token partial slots of the main kernel with diagnostics (kTokPartDiag
// floats per (split, row)); slots 0-2 are sum gate, sum intensity, active count.
constexpr int kTokPartDiag = 12;
enum { TP_SMAX = 4, TP_STRONG, TP_BOUND, TP_075, TP_030, TP_CAP, TP_GLOGG };

// Rows of the main kernel are "virtual tokens" v = t * routes + r: h, tau,
// outputs and every partial are indexed by v, x by v / routes (paired QK runs
// as 2T rows sharing each x row).
// Per-row tau from the moment partials (srw_tau_kernel).
struct TauParams {
  const float* mom;
  const float* tau_off;
  float* tau;
  int64_t T;
  int S_st;
  int64_t N;
  int ms;
  float* token_diag;
  int mode;
  float* sstd;  // [T] s_std per row, or null
  int upp;      // kTauChan: units per partial
};

// The finalize of a call: reduce the N-splits' partials (srw_finalize_kernel).
struct FinalParams {
  const float* out_part;
  const float* tok_part;
  uint16_t* out;         // [T, D] bf16
  float* gate_sum;
  float* den;
  int32_t* n_active;
  int64_t T;
  int D, S, spc;
  int S_tok;             // per-token partial slots in tok_part (S for the fused kernels)
  float scale;
  int tps;               // floats per (split, row) in tok_part: 4, or kTokPartDiag with diagnostics
  const float* tau;      // [T] (diagnostics)
  float* token_diag;     // [T][SRW_TDIAG_COUNT] or null
  GateParams gp;
  float exp_scale;
  int den_gate;          // den = max(sum gate, 1) (the v4.0.1 gate, v401:340)
};

struct MainParams {
  const uint16_t* x;     // [T / routes, D]
  const uint16_t* h;     // [T, dr] (== x when HX)
  int routes;
  const uint16_t* emb;   // [N, dr]
  const uint16_t* read;  // [N, D]
  const uint16_t* wp;    // packed W^T fragments
  const float* tau;      // [T] thresholds (srw_tau_kernel)
  float* out_part;       // [S][T][D]
  float* tok_part;       // [S][T][TPS]: sum gate, sum intensity, active count, - [, diagnostics]
  float2* unit_part;     // [ceil(T / 32)][N] per 32-row block and unit: (sum of scores, max of s - tau),
                         // reduced into unit_diag by srw_unit_diag_kernel (diagnostics) or null
  uint32_t* mask32;      // [T][mask_words32] or null
  int64_t mask_words32;
  Geometry g;
  GateParams gp;
  float exp_scale;       // -sharpness * log2(e)
  int rb;                // decode kernel: row-block groups per split (workgroup = split * rb + group)
  const uint16_t* s_in;  // scores-streaming kernel: the moments kernel's bf16 score buffer
  const float* sstd;     // [T] s_std per row (the v4.0.1 gate) or null
  int gl_raw_bf16;       // the v4.0.1 gate of _srw_inference: s - tau in bf16 (v401:1451-1452)
};

// v4.1 gate of a margin m = s - tau - thr (v41:503-511), with the kernels' operations
__device__ inline float gate_of_margin(float m, const GateParams& gp, float exp_scale) {
  const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(m * exp_scale));
  const float inten = gp.eps + __builtin_amdgcn_fmed3f(m - gp.cut, 0.0f, gp.maxi);
  return act * inten;
}
__device__ inline float gate_of_margin(float m, const MainParams& p) { return gate_of_margin(m, p.gp, p.exp_scale); }

// After reduce_scatter16 over a tile, lanes with bit 4 clear hold one unit
// each (unit unit_of_acc(bitreverse4(lane & 15), half) of the tile): its sum
// of scores and max of s - tau over the wave's 32 rows, stored as one float2
// per (32-row block, unit) -- plain stores, each element written by exactly
// one wave (atomics into unit_diag, 2 x 128 per unit at T = 4096 from every
// CU, doubled the Know-pool main kernel's time).  tw: the wave's first row.
__device__ __attribute__((always_inline)) inline void store_unit_part(const MainParams& p, float su, float mx,
                                                                      int64_t u0, int lane, int half, int64_t lo,
                                                                      int64_t hi, int64_t tw) {
  const int k = 8 * (lane & 1) + 4 * ((lane >> 1) & 1) + 2 * ((lane >> 2) & 1) + ((lane >> 3) & 1);
  const int64_t u = u0 + unit_of_acc(k, half);
  if (p.unit_part && !(lane & 16) && u >= lo && u < hi && tw < p.g.T)
    p.unit_part[(tw >> 5) * p.g.N + u] = make_float2(su, mx);
}

// Training diagnostics of one (token, 32-unit tile) -- the producer-side
// half of the main kernels' DIAG work: per token the max score, act-band
// counts as thresholds on the exp argument (act > 0.9 <=> arg < -log2 9;
// 0.1 < act < 0.9 <=> |arg| < log2 9; 0.05 / 0.95: log2 19; 0.2 / 0.8: 2),
// capped intensities (s >= tau + thr + cut + max_intensity - 1e-3)
// (v41:519-534; the intensity sum and the pass bits come from the gate
// epilogue, as without diagnostics); per unit of the tile the sum of scores
// and the max of s - tau over the wave's 32 rows (v41:445-447, 543-552), by a
// butterfly over the lanes of each half, into unit_part.  sw: the lane's bf16
// scores, element v (unit unit_of_acc(v, half) of its token) in word v / 2,
// the low half for even v.  The tile's unit partials go to an LDS block
// (DiagLds) from which another wave stores them: the storing wave need not
// wait for the stores to complete.
struct DiagLds {
  float2 unit[32];    // per unit of the tile: (sum of scores, max of s - tau) over the block's rows
};
struct TileDiag {
  float smax = -INFINITY;
  uint32_t n_strong = 0, n_bound = 0, n_075 = 0, n_030 = 0, n_cap = 0;
  // FAST: every unit of the tile in [lo, hi) and every row of the wave
  // block valid (the selects drop out)
  template <bool FAST>
  __device__ __attribute__((always_inline)) void tile(const MainParams& p, const uint32_t (&sw)[8], int utile,
                                                      int half, int lane, int64_t lo, int64_t hi, int64_t t,
                                                      float tau_t, DiagLds* dl) {
    const int64_t u0 = static_cast<int64_t>(utile) * kUnitTile;
    const float tau_thr = tau_t + p.gp.thr;
    const float k_exp = -tau_thr * p.exp_scale;
    const float tau_cut = tau_thr + p.gp.cut;
    const float cap_s = tau_cut + (p.gp.maxi - 1e-3f);
    const bool full = FAST || (u0 >= lo && u0 + kUnitTile <= hi);
    float su[16], mx[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float sv = (v & 1) ? hi_f32(sw[v >> 1]) : lo_f32(sw[v >> 1]);
      const int64_t u = u0 + unit_of_acc(v, half);
      const bool uok = full || (u >= lo && u < hi);
      const bool ok = FAST || (t < p.g.T && uok);
      su[v] = ok ? sv : 0.f;
      mx[v] = ok ? sv - tau_t : -INFINITY;
      const float arg = fmaf(sv, p.exp_scale, k_exp);
      const float aa = fabsf(arg);
      smax = fmaxf(smax, uok ? sv : -INFINITY);
      n_strong += (uok && arg < -3.169925001442312f) ? 1u : 0u;
      n_bound += (uok && aa < 3.169925001442312f) ? 1u : 0u;
      n_075 += (uok && aa < 4.247927513443585f) ? 1u : 0u;
      n_030 += (uok && aa < 2.0f) ? 1u : 0u;
      n_cap += (uok && sv >= cap_s) ? 1u : 0u;
    }
    reduce_scatter16(su, lane, [](float x, float y) { return x + y; });
    reduce_scatter16(mx, lane, [](float x, float y) { return fmaxf(x, y); });
    if (!(lane & 16)) {
      const int k = 8 * (lane & 1) + 4 * ((lane >> 1) & 1) + 2 * ((lane >> 2) & 1) + ((lane >> 3) & 1);
      dl->unit[unit_of_acc(k, half)] = make_float2(su[0], mx[0]);
    }
  }
  // a block's unit partials of tile utile from LDS to global memory (lanes
  // 32-63: unit u0 + lane - 32)
  __device__ __attribute__((always_inline)) static void emit(const MainParams& p, const DiagLds* dl, int utile,
                                                             int lane, int64_t lo, int64_t hi, int64_t tw) {
    const int64_t u0 = static_cast<int64_t>(utile) * kUnitTile;
    if (lane >= 32) {
      const int64_t u = u0 + (lane - 32);
      if (p.unit_part && u >= lo && u < hi && tw < p.g.T) p.unit_part[(tw >> 5) * p.g.N + u] = dl->unit[lane - 32];
    }
  }
  // the token's counts over the two lane halves into its partial slots
  __device__ __attribute__((always_inline)) void finish(float* tp, int half, bool row_ok) {
    smax = fmaxf(smax, __shfl_xor(smax, 32));
    n_strong += __shfl_xor(n_strong, 32);
    n_bound += __shfl_xor(n_bound, 32);
    n_075 += __shfl_xor(n_075, 32);
    n_030 += __shfl_xor(n_030, 32);
    n_cap += __shfl_xor(n_cap, 32);
    if (half == 0 && row_ok) {
      tp[TP_SMAX] = smax;
      tp[TP_STRONG] = static_cast<float>(n_strong);
      tp[TP_BOUND] = static_cast<float>(n_bound);
      tp[TP_075] = static_cast<float>(n_075);
      tp[TP_030] = static_cast<float>(n_030);
      tp[TP_CAP] = static_cast<float>(n_cap);
    }
  }
};

// Software pipeline over the split's 32-unit tiles.  Iteration i runs the
// score/read GEMMs of tile i+1 interleaved (sched_group_barrier) with the gate
// epilogue of tile i -- matrix-core and vector-ALU work of one wave overlap --
// then the write GEMM of tile i.  LDS holds two E/R stages (tile i+1 being read,
// tile i+2 being loaded) and two W^T stages (tile i being read, tile i+1
// being loaded): 2 x 48 KB + 2 x 24 KB at d_model = d_route = 384.
template <int DB, int KH, bool HX>
__global__ __launch_bounds__(kThreads, 1) void srw_main_kernel(MainParams p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  constexpr int D = DB * 32;
  constexpr int DR = KH * 16;
  constexpr int KX = D / 16;
  constexpr int F_E = KH, F_R = KX, F_W = 2 * DB;
  constexpr int ER_STAGE = (F_E + F_R) * kFragBytes;
  constexpr int W_STAGE = F_W * kFragBytes;
  static_assert(!HX || KH == KX, "h aliases x only when d_route == d_model");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, col = lane & 31;
  const int split = blockIdx.x % p.g.S;
  const int ttile = blockIdx.x / p.g.S;
  const int64_t tw = static_cast<int64_t>(ttile) * kTokTile + 32 * wave;  // wave's first token
  const int64_t t = tw + col;
  const int64_t tl = t < p.g.T ? t : p.g.T - 1;
  int ta, tb;
  int64_t lo, hi;
  split_range(p.g, p.g.spc, split, ta, tb, lo, hi);

  // token operands, resident for the whole kernel
  u32x4_t xq[KX];
#pragma unroll
  for (int ks = 0; ks < KX; ++ks)
    xq[ks] = *reinterpret_cast<const u32x4_t*>(p.x + (tl / p.routes) * D + 16 * ks + 8 * half);
  u32x4_t hq[HX ? 1 : KH];
  if constexpr (!HX) {
#pragma unroll
    for (int ks = 0; ks < KH; ++ks)
      hq[ks] = *reinterpret_cast<const u32x4_t*>(p.h + tl * DR + 16 * ks + 8 * half);
  }

  const float tau = p.tau[tl];  // srw_tau_kernel (v41:461-464)
  const GateParams gp = p.gp;

  f32x16_t oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};
  float gsum = 0.f, isum = 0.f;
  uint32_t nact = 0;

  char* const er_base = lds;
  char* const w_base = lds + 2 * ER_STAGE;

  // Direct global->LDS loads: wave w issues blocks w, w+4, ... of a group.
  using TileE = RowTile<KH>;
  using TileR = RowTile<KX>;
  const uint32_t lsrc_e[2] = {TileE::lane_src(lane, 0), TileE::lane_src(lane, 1)};
  const uint32_t lsrc_r[2] = {TileR::lane_src(lane, 0), TileR::lane_src(lane, 1)};
  auto issue_er = [&](int tile, int stage) {
    char* sb = er_base + stage * ER_STAGE;
    const int64_t u0 = static_cast<int64_t>(tile) * kUnitTile;
#pragma unroll
    for (int q = 0; q < (F_E + 3) / 4; ++q) {
      const int f = wave + 4 * q;
      if (f < F_E) TileE::load(p.emb, u0, p.g.N, f, lane, lsrc_e, sb);
    }
#pragma unroll
    for (int q = 0; q < (F_R + 3) / 4; ++q) {
      const int f = wave + 4 * q;
      if (f < F_R) TileR::load(p.read, u0, p.g.N, f, lane, lsrc_r, sb + F_E * kFragBytes);
    }
  };
  // LDS offsets of this lane's E / R fragment pieces (see RowTile)
  int le[TileE::NM], lr[TileR::NM];
#pragma unroll
  for (int m = 0; m < TileE::NM; ++m) le[m] = TileE::lane_off(lane, m);
#pragma unroll
  for (int m = 0; m < TileR::NM; ++m) lr[m] = F_E * kFragBytes + TileR::lane_off(lane, m);
  // operand of MFMA k of phase A: HX interleaves score (even k) and read (odd
  // k) steps; otherwise all score steps, then all read steps
  auto er_frag = [&](const char* sbase, int k) {
    const bool is_score = HX ? !(k & 1) : (k < KH);
    const int ks = HX ? (k >> 1) : (k < KH ? k : k - KH);
    const int off = is_score ? le[ks % TileE::NM] + TileE::step_off(ks) : lr[ks % TileR::NM] + TileR::step_off(ks);
    return *reinterpret_cast<const u32x4_t*>(sbase + off);
  };
  auto issue_w = [&](int tile, int stage) {
    char* sb = w_base + stage * W_STAGE;
    const uint16_t* wsrc = p.wp + static_cast<int64_t>(tile) * F_W * 512 + lane * 8;
#pragma unroll
    for (int q = 0; q < (F_W + 3) / 4; ++q) {
      const int f = wave + 4 * q;
      if (f < F_W) g2lds16(wsrc + f * 512, sb + f * kFragBytes);
    }
  };

  // score and read GEMMs of one tile, transposed: rows = units, columns = tokens
  auto phase_a = [&](int stage, f32x16_t& sacc, f32x16_t& racc) {
    const char* base = er_base + stage * ER_STAGE;
    sacc = f32x16_t{};
    racc = f32x16_t{};
    constexpr int NM = KH + KX;
#pragma unroll
    for (int k = 0; k < NM; ++k) {
      const bool is_score = HX ? !(k & 1) : (k < KH);
      const int ks = HX ? (k >> 1) : (k < KH ? k : k - KH);
      if (is_score) sacc = mfma(er_frag(base, k), HX ? xq[ks] : hq[HX ? 0 : ks], sacc);
      else racc = mfma(er_frag(base, k), xq[ks], racc);
    }
  };

  // gate epilogue (v41:503-518): the lane holds token `col` and the 16 units
  // unit_of_acc(v, half); writes the bf16 products packed as the write GEMM's
  // A operand and returns the pass bits (element v at bit 15 - v).
  auto epilogue = [&](auto full_tag, const f32x16_t& sacc, const f32x16_t& racc, int64_t u0,
                      uint32_t* pk) -> uint32_t {
    constexpr bool FULL = decltype(full_tag)::value;
    uint32_t bits = 0;
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      const uint32_t sp = pack_bf16(sacc[v], sacc[v + 1]);   // bf16 scores (v41:503)
      const uint32_t xp = pack_bf16(racc[v], racc[v + 1]);   // bf16 x.r (v41:517)
      float g2[2], in2[2];
      bool on2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float s = e ? hi_f32(sp) : lo_f32(sp);
        const float raw = s - tau;
        const float margin = raw - gp.thr;
        const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(margin * p.exp_scale));
        const float am = fmaxf(margin - gp.cut, 0.0f);
        float inten = gp.eps + fminf(am, gp.maxi);
        float g = act * inten;
        bool on = act > 0.5f;
        if constexpr (!FULL) {
          const int64_t u = u0 + unit_of_acc(v + e, half);
          const bool ok = u >= lo && u < hi;
          g = ok ? g : 0.f;
          inten = ok ? inten : 0.f;
          on = on && ok;
        }
        g2[e] = g;
        in2[e] = inten;
        on2[e] = on;
      }
      gsum += g2[0];
      gsum += g2[1];
      isum += in2[0];
      isum += in2[1];
      bits = (bits << 2) | (on2[0] ? 2u : 0u) | (on2[1] ? 1u : 0u);
      const uint32_t gq = pack_bf16(g2[0], g2[1]);             // gate_bf (v41:516)
      pk[v >> 1] = pack_bf16(lo_f32(gq) * lo_f32(xp), hi_f32(gq) * hi_f32(xp));  // (v41:518)
    }
    return bits;
  };

  // write GEMM: OUT[32 tok x D] += P[32 tok x 32 units] . W_t[32 units x D],
  // W^T fragments read from LDS PF MFMAs ahead
  auto phase_c = [&](int stage, const uint32_t* pk) {
    const char* base = w_base + stage * W_STAGE + lane * 16;
    constexpr int NC = 2 * DB, PF = 4;
    auto frag = [&](int k) {  // MFMA k: j = k / DB, db = k % DB
      return *reinterpret_cast<const u32x4_t*>(base + (2 * (k % DB) + k / DB) * kFragBytes);
    };
    u32x4_t fr[PF];
#pragma unroll
    for (int k = 0; k < PF; ++k) fr[k] = frag(k);
    const u32x4_t a0 = {pk[0], pk[1], pk[2], pk[3]}, a1 = {pk[4], pk[5], pk[6], pk[7]};
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const u32x4_t b = fr[k % PF];
      if (k + PF < NC) fr[k % PF] = frag(k + PF);
      oacc[k % DB] = mfma(k < DB ? a0 : a1, b, oacc[k % DB]);
    }
  };

  // pass bitmask and active count of one tile
  auto emit_mask = [&](int tile, uint32_t bits) {
    const int64_t u0 = static_cast<int64_t>(tile) * kUnitTile;
    const uint32_t b = __builtin_bitreverse32(bits) >> 16;  // element v at bit v
    uint32_t m = (b & 0xFu) | ((b & 0xF0u) << 4) | ((b & 0xF00u) << 8) | ((b & 0xF000u) << 12);
    m <<= 4 * half;
    nact += __builtin_popcount(m);
    m |= __shfl_xor(m, 32);
    if (p.mask32 && half == 0 && t < p.g.T) {
      uint32_t* dst = p.mask32 + t * p.mask_words32 + tile;
      const bool shared = (u0 < lo) || (u0 + kUnitTile > hi && hi < p.g.N);
      if (shared) atomicOr(dst, m);
      else *dst = m;
    }
  };

  // Steady state of the pipeline: the score/read GEMMs of the next tile
  // (NM MFMAs, operands read from LDS PF steps ahead) with the 48 epilogue
  // micro-steps of this tile spread over them; sched_barrier(0) fences each
  // MFMA with its slice so that the wave issues vector work while the matrix
  // core runs.
  auto fused_step = [&](int stage, f32x16_t& sn, f32x16_t& rn, const f32x16_t& sacc,
                        const f32x16_t& racc, uint32_t* pk) -> uint32_t {
    constexpr int NM = KH + KX;
    constexpr int PF = 4;
    const char* base = er_base + stage * ER_STAGE;
    u32x4_t fr[PF];
#pragma unroll
    for (int k = 0; k < PF; ++k) fr[k] = er_frag(base, k);
    sn = f32x16_t{};
    rn = f32x16_t{};
    uint32_t sp[8], xp[8], gpk[8];
    float mg[16], ex[16], gv[16], iv[16];
    bool on[16];
    uint32_t bits = 0;
#pragma unroll
    for (int k = 0; k < NM; ++k) {
      const u32x4_t a = fr[k % PF];
      if (k + PF < NM) fr[k % PF] = er_frag(base, k + PF);
      const bool is_score = HX ? !(k & 1) : (k < KH);
      const int ks = HX ? (k >> 1) : (k < KH ? k : k - KH);
      if (is_score) sn = mfma(a, HX ? xq[ks] : hq[HX ? 0 : ks], sn);
      else rn = mfma(a, xq[ks], rn);
#pragma unroll
      for (int st = (k * 48) / NM; st < ((k + 1) * 48) / NM; ++st) {
        const int typ = kEpiStep[st] >> 4, v = kEpiStep[st] & 15;
        if (typ == 0) {
          if (!(v & 1)) {
            sp[v >> 1] = pack_bf16(sacc[v], sacc[v + 1]);   // bf16 scores (v41:503)
            xp[v >> 1] = pack_bf16(racc[v], racc[v + 1]);   // bf16 x.r (v41:517)
          }
          const float sv = (v & 1) ? hi_f32(sp[v >> 1]) : lo_f32(sp[v >> 1]);
          const float raw = sv - tau;
          mg[v] = raw - gp.thr;
          ex[v] = __builtin_amdgcn_exp2f(mg[v] * p.exp_scale);
        } else if (typ == 1) {
          const float act = __builtin_amdgcn_rcpf(1.0f + ex[v]);
          const float am = fmaxf(mg[v] - gp.cut, 0.0f);
          iv[v] = gp.eps + fminf(am, gp.maxi);
          gv[v] = act * iv[v];
          on[v] = act > 0.5f;
        } else {
          gsum += gv[v];
          isum += iv[v];
          bits = (bits << 1) | (on[v] ? 1u : 0u);
          if (v & 1) {
            gpk[v >> 1] = pack_bf16(gv[v - 1], gv[v]);       // gate_bf (v41:516)
            pk[v >> 1] = pack_bf16(lo_f32(gpk[v >> 1]) * lo_f32(xp[v >> 1]),
                                   hi_f32(gpk[v >> 1]) * hi_f32(xp[v >> 1]));  // (v41:518)
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    return bits;
  };

  // two accumulator pairs alternate between "phase-A results of the tile
  // being finished" and "phase A of the next tile"
  f32x16_t s0 = {}, r0 = {}, s1 = {}, r1 = {};
  if (ta < tb) {
    issue_er(ta, ta & 1);
    issue_w(ta, ta & 1);
    if (ta + 1 < tb) issue_er(ta + 1, (ta + 1) & 1);
    wait_vm0();
    __syncthreads();
    phase_a(ta & 1, s0, r0);
    __syncthreads();
  }
  // one pipeline iteration: finish tile i (its phase-A results in sc/rc)
  // while the next tile's phase A accumulates into sn/rn
  auto iteration = [&](int i, f32x16_t& sc, f32x16_t& rc, f32x16_t& sn, f32x16_t& rn) {
    if (i + 2 < tb) issue_er(i + 2, i & 1);
    if (i + 1 < tb) issue_w(i + 1, (i + 1) & 1);
    const int64_t u0 = static_cast<int64_t>(i) * kUnitTile;
    const bool full = u0 >= lo && u0 + kUnitTile <= hi;
    uint32_t pk[8];
    uint32_t bits;
    if (i + 1 < tb && full) {
      // steady state: next tile's GEMMs overlap this tile's gate epilogue
      bits = fused_step((i + 1) & 1, sn, rn, sc, rc, pk);
    } else {
      if (full) bits = epilogue(std::integral_constant<bool, true>{}, sc, rc, u0, pk);
      else bits = epilogue(std::integral_constant<bool, false>{}, sc, rc, u0, pk);
      if (i + 1 < tb) phase_a((i + 1) & 1, sn, rn);
    }
    phase_c(i & 1, pk);
    emit_mask(i, bits);
    wait_vm0();
    __syncthreads();
  };
  for (int i = ta; i < tb; ++i) {
    iteration(i, s0, r0, s1, r1);
    s0 = s1;
    r0 = r1;
  }

  // partial outputs of this split
  gsum += __shfl_xor(gsum, 32);
  isum += __shfl_xor(isum, 32);
  nact += __shfl_xor(nact, 32);
  if (half == 0 && t < p.g.T) {
    float* tp = p.tok_part + (static_cast<int64_t>(split) * p.g.T + t) * 4;
    tp[0] = gsum;
    tp[1] = isum;
    tp[2] = static_cast<float>(nact);
  }
  float* op = p.out_part + static_cast<int64_t>(split) * p.g.T * D;
  if (tw + 32 <= p.g.T) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) op[(tw + unit_of_acc(v, half)) * D + 32 * db + col] = oacc[db][v];
  } else {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t tt = tw + unit_of_acc(v, half);
        if (tt < p.g.T) op[tt * D + 32 * db + col] = oacc[db][v];
      }
  }
}

// ---------------------------------------------------------------------------
// main, warp-specialised: 8 waves, two per SIMD.  Waves 0-3 (producers) own 32
// tokens each with X (and H) in VGPRs and run the score/read GEMMs of tile i,
// handing the bf16-rounded scores and x.r products (the values the reference
// rounds, v41:503, 517) to LDS.  Waves 4-7 (consumers) own the same 32-token
// blocks: the gate epilogue of tile i - 1 (gate, P, pass bits, sums) in
// registers, then its write GEMM into the fp32 OUT accumulators.  A producer's
// MFMAs thus run back to back while the consumer on the same SIMD issues the
// vector-ALU epilogue beside them.
//
// Per tile two workgroup barriers: the first (mid) lets producers overwrite
// the single score stage S once consumers have read it; the second (end)
// publishes S and the next tile's E/R and W^T.  Both roles issue global->LDS
// loads (producers E/R of the next tile, consumers W^T of this one), spread
// over their compute.  LDS = 2 E/R + 2 W^T stages + S.
// ---------------------------------------------------------------------------
constexpr int kWsThreads = 512;

// DG: training diagnostics -- per-token extras in tok_part (TPS = 12), per-unit
// score sums and max margins per 32-row block into unit_part.  GL: the v4.0.1 GELU
// gate (p.sstd; the row sums carry z+ where v4.1 has the intensity); with DG
// its diagnostics (v401:311-320): the max gate itself in TP_SMAX, the gate >
// 0.5 / boundary / z-band counts, sum g log g, and per unit the max gate in
// place of the max margin.
template <int DB, int KH, bool HX, bool DG, bool GL = false>
__device__ __attribute__((always_inline)) inline void main_ws_body(const MainParams& p, const int bid) {
  // With the GELU gate the producer gates (its registers have room for the
  // longer element chain; the consumer's are held by the write GEMM's
  // accumulators): it hands the consumer bf16(gate) where the scores go,
  // keeps the row sums and emits the pass bits.
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  constexpr int TPS = DG ? kTokPartDiag : 4;
  constexpr int D = DB * 32;
  constexpr int DR = KH * 16;
  constexpr int KX = D / 16;
  constexpr int F_E = KH, F_R = KX, F_W = 2 * DB;
  constexpr int ER_STAGE = (F_E + F_R) * kFragBytes;
  constexpr int W_STAGE = F_W * kFragBytes;
  constexpr int S_BLK = 4 * kFragBytes;  // per token block: bf16 scores (2 KB), bf16 x.r (2 KB)
  static_assert(!HX || KH == KX, "h aliases x only when d_route == d_model");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool producer = wave < 4;
  const int blk = wave & 3;                 // token block of this wave
  const int half = lane >> 5, col = lane & 31;
  const int split = bid % p.g.S;
  const int ttile = bid / p.g.S;
  const int64_t tw = static_cast<int64_t>(ttile) * kTokTile + 32 * blk;
  const int64_t t = tw + col;
  const int64_t tl = t < p.g.T ? t : p.g.T - 1;
  int ta, tb;
  int64_t lo, hi;
  split_range(p.g, p.g.spc, split, ta, tb, lo, hi);
  const int n = tb - ta;

  char* const er_base = lds;
  char* const w_base = lds + 2 * ER_STAGE;
  char* const s_blk = w_base + 2 * W_STAGE + blk * S_BLK + lane * 16;

  // Tile loads, direct global->LDS: each wave a contiguous run of blocks.  A
  // wave's loads are spread over its compute: issued back to back they stall
  // the wave at in-order issue until the memory pipeline drains.
  constexpr int PE = (F_E + 3) / 4, PR = (F_R + 3) / 4, NL_ER = PE + PR;
  constexpr int PW = (F_W + 3) / 4;
  using TileE = RowTile<KH>;
  using TileR = RowTile<KX>;
  const uint32_t lsrc_e[2] = {TileE::lane_src(lane, 0), TileE::lane_src(lane, 1)};
  const uint32_t lsrc_r[2] = {TileR::lane_src(lane, 0), TileR::lane_src(lane, 1)};
  auto er_load = [&](int tile, int stage, int q) {
    char* sb = er_base + stage * ER_STAGE;
    const int64_t u0 = static_cast<int64_t>(tile) * kUnitTile;
    if (q < PE) {
      if (PE * blk + q < F_E) TileE::load(p.emb, u0, p.g.N, PE * blk + q, lane, lsrc_e, sb);
    } else {
      const int r = q - PE;
      if (PR * blk + r < F_R) TileR::load(p.read, u0, p.g.N, PR * blk + r, lane, lsrc_r, sb + F_E * kFragBytes);
    }
  };
  // W^T: wave-uniform tile base + 32-bit lane offset
  const uint32_t w_voff = static_cast<uint32_t>(PW * blk * kFragBytes + lane * 16);
  auto w_load = [&](int tile, int stage, int q) {
    if (PW * blk + q < F_W)
      g2lds16(reinterpret_cast<const char*>(p.wp) + static_cast<int64_t>(tile) * W_STAGE + (w_voff + q * kFragBytes),
              w_base + stage * W_STAGE + (PW * blk + q) * kFragBytes);
  };

  // prologue: E/R of the first tile
  if (n > 0 && producer) {
#pragma unroll
    for (int q = 0; q < NL_ER; ++q) er_load(ta, 0, q);
  }
  wait_vm0();
  __syncthreads();

  if (producer) {
    // ---------------- producer: score / read GEMMs ----------------
    u32x4_t xq[KX];
#pragma unroll
    for (int ks = 0; ks < KX; ++ks)
      xq[ks] = *reinterpret_cast<const u32x4_t*>(p.x + (tl / p.routes) * D + 16 * ks + 8 * half);
    u32x4_t hq[HX ? 1 : KH];
    if constexpr (!HX) {
#pragma unroll
      for (int ks = 0; ks < KH; ++ks)
        hq[ks] = *reinterpret_cast<const u32x4_t*>(p.h + tl * DR + 16 * ks + 8 * half);
    }
    int le[TileE::NM], lr[TileR::NM];  // LDS offsets of this lane's E / R pieces (RowTile)
#pragma unroll
    for (int m = 0; m < TileE::NM; ++m) le[m] = TileE::lane_off(lane, m);
#pragma unroll
    for (int m = 0; m < TileR::NM; ++m) lr[m] = F_E * kFragBytes + TileR::lane_off(lane, m);
    // diagnostics (v41:519-534): the row's max score, act-band counts as
    // thresholds on the exp argument (act > 0.9 <=> arg < -log2 9; 0.1 < act <
    // 0.9 <=> |arg| < log2 9; 0.05 / 0.95: log2 19; 0.2 / 0.8: 2), capped
    // intensities (s >= tau + thr + cut + max_intensity - 1e-3)
    const float tau_t = DG ? p.tau[tl] : 0.f;
    // the GELU gate's row: tau (bf16 for _srw_inference) and 1 / s_std
    const float gl_tau = GL ? (p.gl_raw_bf16 ? __uint_as_float(pack_bf16(0.0f, p.tau[tl])) : p.tau[tl]) : 0.f;
    const float gl_istd = GL ? 1.0f / p.sstd[tl] : 1.f;
    float gl_gsum = 0.f, gl_gmax = 0.f, gl_glogg = 0.f;
    float smax = -INFINITY, isum = 0.f;
    uint32_t n_strong = 0, n_bound = 0, n_075 = 0, n_030 = 0, n_cap = 0, nact = 0;
    // Drain the x / h loads here: left pending into the tile loop, they make
    // the compiler wait for every load in flight (the next tile's LDS
    // prefetch included) at the top of each iteration.
    wait_vm0();
    // diagnostics: a tile's pass-mask word and unit partial are stored at the
    // top of the next iteration, so that the tile's GEMMs cover their latency
    // before the end-of-tile vmcnt wait
    uint32_t pend_m = 0;
    float pend_su = 0.f, pend_mx = 0.f;

    for (int it = 0; it <= n; ++it) {
      if constexpr (DG) {
        if (it >= 1) {
          const int64_t pu0 = static_cast<int64_t>(ta + it - 1) * kUnitTile;
          if (!GL && p.mask32 && half == 0 && t < p.g.T) {  // (the GELU gate stores its mask words at once)
            uint32_t* dst = p.mask32 + t * p.mask_words32 + (ta + it - 1);
            const bool shared = (pu0 < lo) || (pu0 + kUnitTile > hi && hi < p.g.N);
            if (shared) atomicOr(dst, pend_m);
            else *dst = pend_m;
          }
          store_unit_part(p, pend_su, pend_mx, pu0, lane, half, lo, hi, tw);
        }
      }
      const bool pre = it + 1 < n;  // the next tile's E/R go out during this one's MFMAs
      // S piece q (16 B per lane) = bf16 scores and x.r of elements 4q..4q+3:
      // {s[4q], s[4q+1]}, {s[4q+2], s[4q+3]}, {xr[4q], xr[4q+1]}, {xr[4q+2], xr[4q+3]}
      uint32_t sx[16];
      if (it < n) {
        // MFMA k: HX interleaves score (even k) and read (odd k) steps,
        // otherwise all score steps, then all read steps; LDS operands are
        // read PF MFMAs ahead
        const char* base = er_base + (it & 1) * ER_STAGE;
        constexpr int NM = KH + KX, PF = DG ? 4 : 8;
        auto frag = [&](int k) {
          const bool is_score = HX ? !(k & 1) : (k < KH);
          const int ks = HX ? (k >> 1) : (k < KH ? k : k - KH);
          const int off = is_score ? le[ks % TileE::NM] + TileE::step_off(ks)
                                   : lr[ks % TileR::NM] + TileR::step_off(ks);
          return *reinterpret_cast<const u32x4_t*>(base + off);
        };
        u32x4_t fr[PF];
#pragma unroll
        for (int k = 0; k < PF; ++k)
          if (k < NM) fr[k] = frag(k);
        f32x16_t sacc = {}, racc = {};
#pragma unroll
        for (int k = 0; k < NM; ++k) {
#pragma unroll
          for (int q = 0; q < NL_ER; ++q)
            if (k == q * NM / (2 * NL_ER) && pre) er_load(ta + it + 1, (it + 1) & 1, q);  // first half
          const u32x4_t a = fr[k % PF];
          if (k + PF < NM) fr[k % PF] = frag(k + PF);
          const bool is_score = HX ? !(k & 1) : (k < KH);
          const int ks = HX ? (k >> 1) : (k < KH ? k : k - KH);
          if (is_score) sacc = mfma(a, HX ? xq[ks] : hq[HX ? 0 : ks], sacc);
          else racc = mfma(a, xq[ks], racc);
          __builtin_amdgcn_sched_barrier(0);  // keep the reads PF steps ahead
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sx[4 * q] = pack_bf16(sacc[4 * q], sacc[4 * q + 1]);          // bf16 scores (v41:503)
          sx[4 * q + 1] = pack_bf16(sacc[4 * q + 2], sacc[4 * q + 3]);
          sx[4 * q + 2] = pack_bf16(racc[4 * q], racc[4 * q + 1]);      // bf16 x.r (v41:517)
          sx[4 * q + 3] = pack_bf16(racc[4 * q + 2], racc[4 * q + 3]);
        }
        if constexpr (GL) {
          // v4.0.1 gate of the 16 elements (v401:303-310): bf16(gate) replaces
          // the score pairs of sx; gate and z+ sums, pass bits (z > 0)
          const int64_t u0 = static_cast<int64_t>(ta + it) * kUnitTile;
          const bool full = u0 >= lo && u0 + kUnitTile <= hi;
          uint32_t bits = 0;
          [[maybe_unused]] const bool row_ok = t < p.g.T;
          if constexpr (DG) {
            // per unit of the tile the sum of scores over the wave's 32 rows
            // (score_lb, v401:257-260), reduced before the gate loop so that
            // its registers are free there
            float su[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const uint32_t pr = sx[4 * (v >> 2) + ((v & 3) >> 1)];
              const float sv = (v & 1) ? hi_f32(pr) : lo_f32(pr);
              bool ok = row_ok;
              if (!full) {
                const int64_t u = u0 + unit_of_acc(v, half);
                ok = ok && u >= lo && u < hi;
              }
              su[v] = ok ? sv : 0.f;
            }
            reduce_scatter16(su, lane, [](float x, float y) { return x + y; });
            pend_su = su[0];
          }
          // diagnostics: per unit the max gate over the wave's 32 rows
          [[maybe_unused]] float gx[DG ? 16 : 1];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int w = 4 * (q >> 1) + (q & 1);  // the word of elements 2q, 2q + 1
            float g2[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const float sv = e ? hi_f32(sx[w]) : lo_f32(sx[w]);
              float zp;
              float g = gelu_gate(sv, gl_tau, gl_istd, zp, p.gl_raw_bf16 != 0);
              uint32_t sign = __float_as_uint(gl_tau - sv);
              bool ok = true;
              if (!full) {
                const int64_t u = u0 + unit_of_acc(2 * q + e, half);
                ok = u >= lo && u < hi;
                g = ok ? g : 0.f;
                zp = ok ? zp : 0.f;
                sign = ok ? sign : 0u;
              }
              gl_gsum += g;
              isum += zp;
              bits = __builtin_amdgcn_alignbit(bits, sign, 31);  // bits << 1 | active
              g2[e] = g;
              if constexpr (DG) {
                // v401:311-318.  phi > 0.95 or phi < 0.05 <=> |z| > Phi^-1(0.95)
                // (phi is increasing in z; z over every unit, passing or not);
                // 0 < z < 0.75 <=> active and not z+ >= 0.75 (n_075 = active
                // count - those, at the end; likewise 0.30); units outside the
                // split have g = z+ = 0 and are excluded from the boundary
                // count by ok
                const float z = (sv - gl_tau) * gl_istd;
                n_strong += g > 0.5f ? 1u : 0u;
                n_bound += (ok && fabsf(z) > 1.6448536269514722f) ? 1u : 0u;
                n_075 += zp >= 0.75f ? 1u : 0u;
                n_030 += zp >= 0.30f ? 1u : 0u;
                gl_gmax = fmaxf(gl_gmax, g);
                gl_glogg = fmaf(g, __builtin_amdgcn_logf(g + 1e-8f), gl_glogg);  // log2; ln at the end
                gx[2 * q + e] = row_ok ? g : 0.f;
              }
            }
            sx[w] = pack_bf16(g2[0], g2[1]);  // gate_bf (v401:307)
          }
          if constexpr (DG) {
            reduce_scatter16(gx, lane, [](float x, float y) { return fmaxf(x, y); });
            pend_mx = gx[0];
          }
          const uint32_t b = __builtin_bitreverse32(bits) >> 16;  // element v at bit v
          uint32_t m = (b & 0xFu) | ((b & 0xF0u) << 4) | ((b & 0xF00u) << 8) | ((b & 0xF000u) << 12);
          m <<= 4 * half;
          nact += __builtin_popcount(m);
          m |= __shfl_xor(m, 32);
          if (p.mask32 && half == 0 && t < p.g.T) {
            uint32_t* dst = p.mask32 + t * p.mask_words32 + (ta + it);
            const bool shared = (u0 < lo) || (u0 + kUnitTile > hi && hi < p.g.N);
            if (shared) atomicOr(dst, m);
            else *dst = m;
          }
        }
        if constexpr (DG && !GL) {
          // per-unit sum of scores and max of (score - tau) over this wave's 32
          // rows (v41:445-447, 543-552): butterfly over the lanes of each half
          const int64_t u0 = static_cast<int64_t>(ta + it) * kUnitTile;
          const float tau_thr = tau_t + p.gp.thr;
          const float k_exp = -tau_thr * p.exp_scale;
          const float tau_cut = tau_thr + p.gp.cut;
          const float cap_s = tau_cut + (p.gp.maxi - 1e-3f);
          const bool full = u0 >= lo && u0 + kUnitTile <= hi;
          const bool row_ok = t < p.g.T;
          uint32_t bits = 0;
          float su[16], mx[16];
          // A unit outside [lo, hi), or a row past T, enters as score -inf:
          // no band, pass bit, cap or max score counts it (exp argument
          // +inf); only its score sum and intensity need a select.
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const uint32_t pr = sx[4 * (v >> 2) + ((v & 3) >> 1)];
            const float s_raw = (v & 1) ? hi_f32(pr) : lo_f32(pr);
            const int64_t u = u0 + unit_of_acc(v, half);
            const bool ok = row_ok && (full || (u >= lo && u < hi));
            const float sv = ok ? s_raw : -INFINITY;
            su[v] = ok ? s_raw : 0.f;
            mx[v] = sv - tau_t;
            const float arg = fmaf(sv, p.exp_scale, k_exp);
            const float aa = fabsf(arg);
            smax = fmaxf(smax, sv);
            n_strong += arg < -3.169925001442312f ? 1u : 0u;
            n_bound += aa < 3.169925001442312f ? 1u : 0u;
            n_075 += aa < 4.247927513443585f ? 1u : 0u;
            n_030 += aa < 2.0f ? 1u : 0u;
            n_cap += sv >= cap_s ? 1u : 0u;
            // intensity sum and pass bits (v41:503-511, 528) as in the gate epilogue
            const float inten = p.gp.eps + __builtin_amdgcn_fmed3f(sv - tau_cut, 0.0f, p.gp.maxi);
            isum += ok ? inten : 0.f;
            bits = __builtin_amdgcn_alignbit(bits, __float_as_uint(arg), 31);
          }
          {
            const uint32_t b = __builtin_bitreverse32(bits) >> 16;  // element v at bit v
            uint32_t m = (b & 0xFu) | ((b & 0xF0u) << 4) | ((b & 0xF00u) << 8) | ((b & 0xF000u) << 12);
            m <<= 4 * half;
            nact += __builtin_popcount(m);
            pend_m = m | __shfl_xor(m, 32);
          }
          reduce_scatter16(su, lane, [](float x, float y) { return x + y; });
          reduce_scatter16(mx, lane, [](float x, float y) { return fmaxf(x, y); });
          pend_su = su[0];
          pend_mx = mx[0];
        }
      }
      barrier_lds();  // mid: consumers have read S (tile it - 1)
      if (it < n) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<u32x4_t*>(s_blk + q * kFragBytes) =
              u32x4_t{sx[4 * q], sx[4 * q + 1], sx[4 * q + 2], sx[4 * q + 3]};
      }
      wait_vm0();
      barrier_lds();  // end: S, next E/R and W^T visible
    }
    if constexpr (GL) {
      gl_gsum += __shfl_xor(gl_gsum, 32);
      isum += __shfl_xor(isum, 32);
      nact += __shfl_xor(nact, 32);
      if constexpr (DG) {
        gl_gmax = fmaxf(gl_gmax, __shfl_xor(gl_gmax, 32));
        n_strong += __shfl_xor(n_strong, 32);
        n_bound += __shfl_xor(n_bound, 32);
        n_075 += __shfl_xor(n_075, 32);
        n_030 += __shfl_xor(n_030, 32);
        gl_glogg += __shfl_xor(gl_glogg, 32);
      }
      if (half == 0 && t < p.g.T) {
        float* tp = p.tok_part + (static_cast<int64_t>(split) * p.g.T + t) * TPS;
        tp[0] = gl_gsum;
        tp[1] = isum;  // sum of z+
        tp[2] = static_cast<float>(nact);
        if constexpr (DG) {
          tp[TP_SMAX] = gl_gmax;  // the max gate itself
          tp[TP_STRONG] = static_cast<float>(n_strong);
          tp[TP_BOUND] = static_cast<float>(n_bound);
          tp[TP_075] = static_cast<float>(nact - n_075);  // 0 < z < 0.75
          tp[TP_030] = static_cast<float>(nact - n_030);
          tp[TP_CAP] = 0.f;
          tp[TP_GLOGG] = gl_glogg * 0.69314718055994531f;  // log2 -> ln
        }
      }
    }
    if constexpr (DG && !GL) {
      smax = fmaxf(smax, __shfl_xor(smax, 32));
      n_strong += __shfl_xor(n_strong, 32);
      n_bound += __shfl_xor(n_bound, 32);
      n_075 += __shfl_xor(n_075, 32);
      n_030 += __shfl_xor(n_030, 32);
      n_cap += __shfl_xor(n_cap, 32);
      isum += __shfl_xor(isum, 32);
      nact += __shfl_xor(nact, 32);
      if (half == 0 && t < p.g.T) {
        float* tp = p.tok_part + (static_cast<int64_t>(split) * p.g.T + t) * TPS;
        tp[1] = isum;
        tp[2] = static_cast<float>(nact);
        tp[TP_SMAX] = smax;
        tp[TP_STRONG] = static_cast<float>(n_strong);
        tp[TP_BOUND] = static_cast<float>(n_bound);
        tp[TP_075] = static_cast<float>(n_075);
        tp[TP_030] = static_cast<float>(n_030);
        tp[TP_CAP] = static_cast<float>(n_cap);
      }
    }
  } else {
    // ---------------- consumer: gate epilogue and write GEMM, one tile behind ----------------
    // tau = mean + tau_offset * (sqrt(E[s^2] - mean^2) + 1e-8) (v41:461-464,
    // srw_tau_kernel), folded with the gate's constant offsets:
    //   margin = s - tau - thr,  exp argument = margin * c  (c = -sharpness log2 e)
    float k_exp, tau_cut;
    {
      const float tau_thr = p.tau[tl] + p.gp.thr;
      k_exp = -tau_thr * p.exp_scale;
      tau_cut = tau_thr + p.gp.cut;
    }
    const float c_exp = p.exp_scale, eps = p.gp.eps, maxi = p.gp.maxi;
    float gsum = 0.f, isum = 0.f;
    uint32_t nact = 0;
    float glogg = 0.f;  // diagnostics: sum gate * log2(gate + 1e-8) (v41:533-534)
    f32x16_t oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};
    wait_vm0();

    // gate epilogue (v41:503-518) of one tile from the bf16 scores / x.r:
    // P (the write GEMM's A operand, k-step j in pk[4j..4j+3]) and the pass
    // bits (element v at bit 15 - v); W^T loads of the tile go out between
    // element pairs
    auto gate_tile = [&](auto full_tag, int64_t u0, uint32_t* pk, int wtile, int wstage) -> uint32_t {
      constexpr bool FULL = decltype(full_tag)::value;
      uint32_t bits = 0;
      u32x4_t sq;
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        if ((v & 3) == 0) sq = *reinterpret_cast<const u32x4_t*>(s_blk + (v >> 2) * kFragBytes);
        if ((v >> 1) < PW && wtile >= 0) w_load(wtile, wstage, v >> 1);
        const uint32_t sp = sq[(v >> 1) & 1], xp = sq[2 + ((v >> 1) & 1)];
        if constexpr (GL) {
          // the producer's bf16 gate pair in place of the scores
          pk[v >> 1] = pack_bf16(lo_f32(sp) * lo_f32(xp), hi_f32(sp) * hi_f32(xp));  // (v401:309)
          continue;
        }
        float g2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float sv = e ? hi_f32(sp) : lo_f32(sp);
          // sigmoid(sharpness * margin) = 1 / (1 + 2^(margin * c)); active <=> margin > 0 <=> arg < 0
          const float arg = fmaf(sv, c_exp, k_exp);
          const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(arg));
          // intensity = eps + min(max(margin - cutoff, 0), max_intensity)
          float inten = eps + __builtin_amdgcn_fmed3f(sv - tau_cut, 0.0f, maxi);
          float g = act * inten;
          uint32_t sign = __float_as_uint(arg);
          if constexpr (!FULL) {
            const int64_t u = u0 + unit_of_acc(v + e, half);
            const bool ok = u >= lo && u < hi;
            g = ok ? g : 0.f;
            inten = ok ? inten : 0.f;
            sign = ok ? sign : 0u;
          }
          gsum += g;
          if constexpr (DG) {
            glogg = fmaf(g, __builtin_amdgcn_logf(g + 1e-8f), glogg);
          } else {
            isum += inten;
            bits = __builtin_amdgcn_alignbit(bits, sign, 31);   // bits << 1 | active
          }
          g2[e] = g;
        }
        const uint32_t gq = pack_bf16(g2[0], g2[1]);             // gate_bf (v41:516)
        pk[v >> 1] = pack_bf16(lo_f32(gq) * lo_f32(xp), hi_f32(gq) * hi_f32(xp));  // (v41:518)
      }
      return bits;
    };

    for (int it = 0; it <= n; ++it) {
      const bool cur = it < n;  // this tile's W^T goes out during the previous tile's epilogue
      if (it == 0) {
        if (cur) {
#pragma unroll
          for (int q = 0; q < PW; ++q) w_load(ta, 0, q);
        }
        barrier_lds();  // mid
      } else {
        const int tile = ta + it - 1;
        const int64_t u0 = static_cast<int64_t>(tile) * kUnitTile;
        uint32_t pk[8];
        uint32_t bits;
        const int wtile = cur ? ta + it : -1;
        if (u0 >= lo && u0 + kUnitTile <= hi)
          bits = gate_tile(std::integral_constant<bool, true>{}, u0, pk, wtile, it & 1);
        else
          bits = gate_tile(std::integral_constant<bool, false>{}, u0, pk, wtile, it & 1);
        // pass bitmask of the tile (the producer emits it with diagnostics and
        // the GELU gate)
        if constexpr (!DG && !GL) {
          const uint32_t b = __builtin_bitreverse32(bits) >> 16;  // element v at bit v
          uint32_t m = (b & 0xFu) | ((b & 0xF0u) << 4) | ((b & 0xF00u) << 8) | ((b & 0xF000u) << 12);
          m <<= 4 * half;
          nact += __builtin_popcount(m);
          m |= __shfl_xor(m, 32);
          if (p.mask32 && half == 0 && t < p.g.T) {
            uint32_t* dst = p.mask32 + t * p.mask_words32 + tile;
            const bool shared = (u0 < lo) || (u0 + kUnitTile > hi && hi < p.g.N);
            if (shared) atomicOr(dst, m);
            else *dst = m;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        // write GEMM: OUT[32 tok x D] += P[32 tok x 32 units] . W_t[32 units x D]
        const char* wb = w_base + ((it - 1) & 1) * W_STAGE + lane * 16;
        const u32x4_t a0 = {pk[0], pk[1], pk[2], pk[3]}, a1 = {pk[4], pk[5], pk[6], pk[7]};
        constexpr int NC = 2 * DB, PF = DG ? 4 : 6;
        auto frag = [&](int k) {  // MFMA k: j = k / DB, db = k % DB
          return *reinterpret_cast<const u32x4_t*>(wb + (2 * (k % DB) + k / DB) * kFragBytes);
        };
        u32x4_t fr[PF];
#pragma unroll
        for (int k = 0; k < PF; ++k)
          if (k < NC) fr[k] = frag(k);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          const u32x4_t bq = fr[k % PF];
          if (k + PF < NC) fr[k % PF] = frag(k + PF);
          oacc[k % DB] = mfma(k < DB ? a0 : a1, bq, oacc[k % DB]);
          __builtin_amdgcn_sched_barrier(0);
        }
        barrier_lds();  // mid
      }
      wait_vm0();
      barrier_lds();  // end
    }
    gsum += __shfl_xor(gsum, 32);
    isum += __shfl_xor(isum, 32);
    nact += __shfl_xor(nact, 32);
    if constexpr (DG) glogg += __shfl_xor(glogg, 32);
    if (!GL && half == 0 && t < p.g.T) {  // the producer has the GELU gate's sums
      float* tp = p.tok_part + (static_cast<int64_t>(split) * p.g.T + t) * TPS;
      tp[0] = gsum;
      if constexpr (DG) {
        tp[TP_GLOGG] = glogg * 0.69314718055994531f;  // log2 -> ln
      } else {
        tp[1] = isum;
        tp[2] = static_cast<float>(nact);
      }
    }
    float* op = p.out_part + static_cast<int64_t>(split) * p.g.T * D;
    if (tw + 32 <= p.g.T) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) op[(tw + unit_of_acc(v, half)) * D + 32 * db + col] = oacc[db][v];
    } else {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t tt = tw + unit_of_acc(v, half);
          if (tt < p.g.T) op[tt * D + 32 * db + col] = oacc[db][v];
        }
    }
  }
}

template <int DB, int KH, bool HX, bool DG, bool GL = false>
__global__ __launch_bounds__(kWsThreads, 1) void srw_main_ws_kernel(MainParams p) {
  main_ws_body<DB, KH, HX, DG, GL>(p, blockIdx.x);
}
template <int DB, int KH, bool HX>
__global__ __launch_bounds__(kWsThreads, 1) void srw_main_ws_batch_kernel(Batch<MainParams> b) {
  const int i = batch_index(b.start, b.n, blockIdx.x);
  main_ws_body<DB, KH, HX, false>(b.p[i], blockIdx.x - b.start[i]);
}

// ---------------------------------------------------------------------------
// main, scores streamed: the warp-specialised layout of srw_main_ws_kernel
// with the bf16 scores read back from the moments kernel's score buffer
// (kScoreTileBytes per (token tile, unit tile)) instead of recomputed -- the
// same bf16 values: the same fragments, MFMA and k order produced them.
// Producers (waves 0-3) run only the read GEMM XR^T = R_t.X^T, hand the
// bf16 x.r (v41:517) to a double-buffered LDS stage, and issue every load of
// the workgroup beside their MFMAs: the next tile's R, this tile's W^T and
// the consumers' 32 x 32 score blocks (2 KB per token block; the producers'
// MFMA stream has the slack, the consumers' epilogue is the critical path).
// Consumers (waves 4-7) run the gate epilogue of the previous tile and its
// write GEMM, and never wait for memory.  With every stage doubled one
// workgroup barrier per tile suffices: a stage is rewritten two tiles after
// it was filled, past the barrier that ends the reads of it.  LDS = 2 R +
// 2 W^T + 2 x.r + 2 score stages (128 KB at d_model = 384).
// ---------------------------------------------------------------------------
template <int DB, bool DG = false>
constexpr int ss_lds_bytes() {
  return (2 * (DB * 2) + 2 * (2 * DB) + 2 * 8 + 2 * 8) * kFragBytes + (DG ? 2 * 4 * static_cast<int>(sizeof(DiagLds)) : 0);
}

// DG: training diagnostics, split as in srw_main_ws_kernel -- the producers
// take the per-token counts, pass bits and per-unit statistics of the tile
// the consumers gate (from the same score stage, one tile behind their own
// read GEMM), the consumers the gate sum and sum gate log gate.
template <int DB, bool DG = false>
__device__ __attribute__((always_inline)) inline void main_ss_body(const MainParams& p, const int bid) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  constexpr int TPS = DG ? kTokPartDiag : 4;
  constexpr int D = DB * 32;
  constexpr int KX = D / 16;
  constexpr int F_R = KX, F_W = 2 * DB;
  constexpr int R_STAGE = F_R * kFragBytes;
  constexpr int W_STAGE = F_W * kFragBytes;
  constexpr int XR_BLK = 2 * kFragBytes;  // per token block: bf16 x.r (2 KB)
  constexpr int XR_STAGE = 4 * XR_BLK;
  constexpr int S_BLK = 2 * kFragBytes;   // per token block: bf16 scores (2 KB)
  constexpr int S_STAGE = 4 * S_BLK;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool producer = wave < 4;
  const int blk = wave & 3;                 // token block of this wave
  const int half = lane >> 5, col = lane & 31;
  const int split = bid % p.g.S;
  const int ttile = bid / p.g.S;
  const int64_t tw = static_cast<int64_t>(ttile) * kTokTile + 32 * blk;
  const int64_t t = tw + col;
  const int64_t tl = t < p.g.T ? t : p.g.T - 1;
  int ta, tb;
  int64_t lo, hi;
  split_range(p.g, p.g.spc, split, ta, tb, lo, hi);
  const int n = tb - ta;

  char* const r_base = lds;
  char* const w_base = lds + 2 * R_STAGE;
  char* const xr_lane = w_base + 2 * W_STAGE + blk * XR_BLK + lane * 16;  // + stage * XR_STAGE
  char* const s_wave = w_base + 2 * W_STAGE + 2 * XR_STAGE + blk * S_BLK;  // + stage * S_STAGE
  // diagnostics: the producers' mask words and unit partials of a tile, which
  // the consumers store one tile later ([stage][block])
  DiagLds* const d_blk = reinterpret_cast<DiagLds*>(w_base + 2 * W_STAGE + 2 * XR_STAGE + 2 * S_STAGE) + blk;

  // R and W^T tiles, direct global->LDS, each wave a contiguous run of blocks
  constexpr int PR = (F_R + 3) / 4, PW = (F_W + 3) / 4;
  using TileR = RowTile<KX>;
  const uint32_t lsrc_r[2] = {TileR::lane_src(lane, 0), TileR::lane_src(lane, 1)};
  auto r_load = [&](int tile, int stage, int q) {
    if (PR * blk + q < F_R)
      TileR::load(p.read, static_cast<int64_t>(tile) * kUnitTile, p.g.N, PR * blk + q, lane, lsrc_r,
                  r_base + stage * R_STAGE);
  };
  const uint32_t w_voff = static_cast<uint32_t>(PW * blk * kFragBytes + lane * 16);
  auto w_load = [&](int tile, int stage, int q) {
    if (PW * blk + q < F_W)
      g2lds16(reinterpret_cast<const char*>(p.wp) + static_cast<int64_t>(tile) * W_STAGE + (w_voff + q * kFragBytes),
              w_base + stage * W_STAGE + (PW * blk + q) * kFragBytes);
  };

  // this wave's score blocks: tile u at s_src + u * kScoreTileBytes (elements 0-7), + 1 KB (8-15)
  const char* const s_src =
      reinterpret_cast<const char*>(p.s_in) + score_tile_off(p.g.ntiles, ttile, 0, blk) + lane * 16;
  auto s_load = [&](int tile, int stage) {
    const char* src = s_src + static_cast<int64_t>(tile) * kScoreTileBytes;
    g2lds16_nt(src, s_wave + stage * S_STAGE);  // read once
    g2lds16_nt(src + kFragBytes, s_wave + stage * S_STAGE + kFragBytes);
  };

  // prologue: R of the first tile
  if (n > 0 && producer) {
#pragma unroll
    for (int q = 0; q < PR; ++q) r_load(ta, 0, q);
  }
  wait_vm0();
  __syncthreads();

  if (producer) {
    // ---------------- producer: read GEMM ----------------
    u32x4_t xq[KX];
#pragma unroll
    for (int ks = 0; ks < KX; ++ks)
      xq[ks] = *reinterpret_cast<const u32x4_t*>(p.x + (tl / p.routes) * D + 16 * ks + 8 * half);
    int lr[TileR::NM];
#pragma unroll
    for (int m = 0; m < TileR::NM; ++m) lr[m] = TileR::lane_off(lane, m);
    wait_vm0();  // x drained here, not at the first tile's vmcnt wait
    TileDiag dgs;                            // diagnostics
    const float tau_t = DG ? p.tau[tl] : 0.f;

    for (int it = 0; it <= n; ++it) {
      if constexpr (DG) {
        // diagnostics of the tile the consumers gate now (its scores came in
        // with the previous tile's loads)
        if (it >= 1) {
          const char* sb = s_wave + ((it - 1) & 1) * S_STAGE + lane * 16;
          const u32x4_t s0 = *reinterpret_cast<const u32x4_t*>(sb);
          const u32x4_t s1 = *reinterpret_cast<const u32x4_t*>(sb + kFragBytes);
          const uint32_t sw[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
          const int64_t u0 = static_cast<int64_t>(ta + it - 1) * kUnitTile;
          if (u0 >= lo && u0 + kUnitTile <= hi && tw + 32 <= p.g.T)
            dgs.tile<true>(p, sw, ta + it - 1, half, lane, lo, hi, t, tau_t, d_blk + ((it - 1) & 1) * 4);
          else
            dgs.tile<false>(p, sw, ta + it - 1, half, lane, lo, hi, t, tau_t, d_blk + ((it - 1) & 1) * 4);
        }
      }
      if (it < n) {
        const bool pre = it + 1 < n;  // the next tile's R goes out during this one's MFMAs
        const char* base = r_base + (it & 1) * R_STAGE;
        constexpr int PF = 8;
        auto frag = [&](int k) {
          return *reinterpret_cast<const u32x4_t*>(base + lr[k % TileR::NM] + TileR::step_off(k));
        };
        u32x4_t fr[PF];
#pragma unroll
        for (int k = 0; k < PF; ++k)
          if (k < KX) fr[k] = frag(k);
        f32x16_t racc = {};
#pragma unroll
        for (int k = 0; k < KX; ++k) {
#pragma unroll
          for (int q = 0; q < PR; ++q)
            if (k == q * KX / (2 * PR) && pre) r_load(ta + it + 1, (it + 1) & 1, q);  // first half
          // this tile's W^T and scores, for the consumers' next iteration
#pragma unroll
          for (int q = 0; q < PW; ++q)
            if (k == KX / 2 + q * (KX / 2 - 1) / (PW + 1)) w_load(ta + it, it & 1, q);
          if (k == KX - 1) s_load(ta + it, it & 1);
          const u32x4_t a = fr[k % PF];
          if (k + PF < KX) fr[k % PF] = frag(k + PF);
          racc = mfma(a, xq[k], racc);
          __builtin_amdgcn_sched_barrier(0);  // keep the reads PF steps ahead
        }
        uint32_t xr[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) xr[q] = pack_bf16(racc[2 * q], racc[2 * q + 1]);  // bf16 x.r (v41:517)
        char* dst = xr_lane + (it & 1) * XR_STAGE;
        *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{xr[0], xr[1], xr[2], xr[3]};
        *reinterpret_cast<u32x4_t*>(dst + kFragBytes) = u32x4_t{xr[4], xr[5], xr[6], xr[7]};
      }
      wait_vm0();
      barrier_lds();  // x.r of this tile, the next tile's R and W^T visible
    }
    if constexpr (DG) dgs.finish(p.tok_part + (static_cast<int64_t>(split) * p.g.T + t) * TPS, half, t < p.g.T);
  } else {
    // ---------------- consumer: gate epilogue and write GEMM, one tile behind ----------------
    // tau folded with the gate's constant offsets (srw_main_ws_kernel):
    //   margin = s - tau - thr,  exp argument = margin * c  (c = -sharpness log2 e)
    float k_exp, tau_cut;
    {
      const float tau_thr = p.tau[tl] + p.gp.thr;
      k_exp = -tau_thr * p.exp_scale;
      tau_cut = tau_thr + p.gp.cut;
    }
    const float c_exp = p.exp_scale, eps = p.gp.eps, maxi = p.gp.maxi;
    float gsum = 0.f, isum = 0.f;
    uint32_t nact = 0;
    float glogg = 0.f;  // diagnostics: sum gate * log2(gate + 1e-8) (v41:533-534)
    f32x16_t oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] = f32x16_t{};
    // gate epilogue (v41:503-518) of one tile from its bf16 scores and x.r
    // (LDS): P (k-step j in pk[4j..4j+3]) and the pass bits (element v at bit
    // 15 - v)
    auto gate_tile = [&](auto full_tag, int64_t u0, uint32_t* pk, const char* srp, const char* xrp) -> uint32_t {
      constexpr bool FULL = decltype(full_tag)::value;
      uint32_t bits = 0;
      u32x4_t sq, xq4;
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        if ((v & 7) == 0) {
          sq = *reinterpret_cast<const u32x4_t*>(srp + (v >> 3) * kFragBytes);
          xq4 = *reinterpret_cast<const u32x4_t*>(xrp + (v >> 3) * kFragBytes);
        }
        const uint32_t sp = sq[(v >> 1) & 3];
        const uint32_t xp = xq4[(v >> 1) & 3];
        float g2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float sv = e ? hi_f32(sp) : lo_f32(sp);
          // sigmoid(sharpness * margin) = 1 / (1 + 2^(margin * c)); active <=> margin > 0 <=> arg < 0
          const float arg = fmaf(sv, c_exp, k_exp);
          const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(arg));
          // intensity = eps + min(max(margin - cutoff, 0), max_intensity)
          float inten = eps + __builtin_amdgcn_fmed3f(sv - tau_cut, 0.0f, maxi);
          float g = act * inten;
          uint32_t sign = __float_as_uint(arg);
          if constexpr (!FULL) {
            const int64_t u = u0 + unit_of_acc(v + e, half);
            const bool ok = u >= lo && u < hi;
            g = ok ? g : 0.f;
            inten = ok ? inten : 0.f;
            sign = ok ? sign : 0u;
          }
          gsum += g;
          if constexpr (DG) glogg = fmaf(g, __builtin_amdgcn_logf(g + 1e-8f), glogg);  // sum gate log2 (gate + 1e-8)
          isum += inten;
          bits = __builtin_amdgcn_alignbit(bits, sign, 31);   // bits << 1 | active
          g2[e] = g;
        }
        const uint32_t gq = pack_bf16(g2[0], g2[1]);             // gate_bf (v41:516)
        pk[v >> 1] = pack_bf16(lo_f32(gq) * lo_f32(xp), hi_f32(gq) * hi_f32(xp));  // (v41:518)
      }
      return bits;
    };

    // the producers load every tile (R, W^T, scores): a consumer's global
    // accesses are its mask words and partials, stores it need not wait for
    for (int it = 0; it <= n; ++it) {
      // diagnostics: the producers' unit partials of tile ta + it - 2
      // (written in the previous iteration)
      if constexpr (DG)
        if (it >= 2) TileDiag::emit(p, d_blk + (it & 1) * 4, ta + it - 2, lane, lo, hi, tw);
      if (it > 0) {
        const int tile = ta + it - 1;
        const int64_t u0 = static_cast<int64_t>(tile) * kUnitTile;
        const char* srp = s_wave + ((it - 1) & 1) * S_STAGE + lane * 16;
        const char* xrp = xr_lane + ((it - 1) & 1) * XR_STAGE;
        uint32_t pk[8];
        uint32_t bits;
        if (u0 >= lo && u0 + kUnitTile <= hi)
          bits = gate_tile(std::integral_constant<bool, true>{}, u0, pk, srp, xrp);
        else
          bits = gate_tile(std::integral_constant<bool, false>{}, u0, pk, srp, xrp);
        // pass bitmask of the tile
        {
          const uint32_t b = __builtin_bitreverse32(bits) >> 16;  // element v at bit v
          uint32_t m = (b & 0xFu) | ((b & 0xF0u) << 4) | ((b & 0xF00u) << 8) | ((b & 0xF000u) << 12);
          m <<= 4 * half;
          nact += __builtin_popcount(m);
          m |= __shfl_xor(m, 32);
          if (p.mask32 && half == 0 && t < p.g.T) {
            uint32_t* dst = p.mask32 + t * p.mask_words32 + tile;
            const bool shared = (u0 < lo) || (u0 + kUnitTile > hi && hi < p.g.N);
            if (shared) atomicOr(dst, m);
            else *dst = m;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        // write GEMM: OUT[32 tok x D] += P[32 tok x 32 units] . W_t[32 units x D]
        const char* wb = w_base + ((it - 1) & 1) * W_STAGE + lane * 16;
        const u32x4_t a0 = {pk[0], pk[1], pk[2], pk[3]}, a1 = {pk[4], pk[5], pk[6], pk[7]};
        constexpr int NC = 2 * DB, PF = 4;
        auto frag = [&](int k) {  // MFMA k: j = k / DB, db = k % DB
          return *reinterpret_cast<const u32x4_t*>(wb + (2 * (k % DB) + k / DB) * kFragBytes);
        };
        u32x4_t fr[PF];
#pragma unroll
        for (int k = 0; k < PF; ++k)
          if (k < NC) fr[k] = frag(k);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          const u32x4_t bq = fr[k % PF];
          if (k + PF < NC) fr[k % PF] = frag(k + PF);
          oacc[k % DB] = mfma(k < DB ? a0 : a1, bq, oacc[k % DB]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      barrier_lds();
    }
    if constexpr (DG)
      if (n >= 1) TileDiag::emit(p, d_blk + ((n + 1) & 1) * 4, ta + n - 1, lane, lo, hi, tw);
    gsum += __shfl_xor(gsum, 32);
    isum += __shfl_xor(isum, 32);
    nact += __shfl_xor(nact, 32);
    if constexpr (DG) glogg += __shfl_xor(glogg, 32);
    if (half == 0 && t < p.g.T) {
      float* tp = p.tok_part + (static_cast<int64_t>(split) * p.g.T + t) * TPS;
      tp[0] = gsum;
      tp[1] = isum;
      tp[2] = static_cast<float>(nact);
      if constexpr (DG) tp[TP_GLOGG] = glogg * 0.69314718055994531f;  // log2 -> ln
    }
    float* op = p.out_part + static_cast<int64_t>(split) * p.g.T * D;
    if (tw + 32 <= p.g.T) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) op[(tw + unit_of_acc(v, half)) * D + 32 * db + col] = oacc[db][v];
    } else {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t tt = tw + unit_of_acc(v, half);
          if (tt < p.g.T) op[tt * D + 32 * db + col] = oacc[db][v];
        }
    }
  }
}

template <int DB, bool DG = false>
__global__ __launch_bounds__(kWsThreads, 1) void srw_main_ss_kernel(MainParams p) {
  main_ss_body<DB, DG>(p, blockIdx.x);
}
template <int DB>
__global__ __launch_bounds__(kWsThreads, 1) void srw_main_ss_batch_kernel(Batch<MainParams> b) {
  const int i = batch_index(b.start, b.n, blockIdx.x);
  main_ss_body<DB>(b.p[i], blockIdx.x - b.start[i]);
}

// ---------------------------------------------------------------------------
// tau: per row, the moment partials -> tau = mean + tau_offset * (sqrt(E[s^2]
// - mean^2) + 1e-8) (v41:461-464).  One wave per row; lanes split the
// partials.  mom holds ms floats per (split, row): s, s^2 [, s^3, s^4].  With
// token_diag, also the row's mean, std, tau and third / fourth power sums
// (zero without them).
// ---------------------------------------------------------------------------
// mode kTauOnePass: std = sqrt(E[s^2] - mean^2) + 1e-8; kTauChan: std =
// sqrt(M2 / N) + 1e-8 (v41:1719-1721) with M2 the partials' centred sums of
// squares merged by Chan et al.'s formula.
// Row t's statistics from the moment partials mom[S_st][T][ms], by one wave:
// the lanes stride over the partials in a fixed order and a fixed butterfly
// joins them.  Up to 256 partials (every decode and fused prefill call) a
// lane's (at most four) partials are loaded at once, one round trip instead
// of a chain of dependent loads; the sums keep the loop's order (the same
// bits).
struct TauRow {
  float mean, sd, tv, c, d;  // c, d: the row's sums of s^3, s^4 (ms == 4)
};
__device__ __attribute__((always_inline)) inline TauRow tau_row(const TauParams& q, const int64_t t, const int lane) {
  const int64_t T = q.T, N = q.N;
  const int S_st = q.S_st, ms = q.ms, mode = q.mode;
  const float* __restrict__ mcol = q.mom + t * ms;  // partial s at mcol + s * T * ms
  const int64_t sstr = T * ms;
  // the partial's unit count (kTauChan): the third float, or from upp
  auto count_of = [&](int s, float stored) {
    if (q.upp <= 0) return stored;
    const int64_t left = N - static_cast<int64_t>(s) * q.upp;
    return static_cast<float>(left <= 0 ? 0 : (left < q.upp ? left : q.upp));
  };
  float a = 0.f, b = 0.f, c = 0.f, d = 0.f;
  if (S_st <= 256) {
    // (no branches around the loads: lanes past S_st load the last partial
    // and add +0, which leaves a sum's bits unchanged)
    float v0[4], v1[4], v2[4], v3[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = lane + 64 * j < S_st ? lane + 64 * j : S_st - 1;
      const float* m = mcol + s * sstr;
      v0[j] = m[0];
      v1[j] = m[1];
      v2[j] = ms >= 3 ? m[2] : 0.f;
      v3[j] = ms == 4 ? m[3] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = lane + 64 * j < S_st;
      a += in ? v0[j] : 0.f;
      b += in ? v1[j] : 0.f;
      if (ms == 4) {
        c += in ? v2[j] : 0.f;
        d += in ? v3[j] : 0.f;
      }
    }
    a = wave_sum(a);
    if (mode == kTauChan) {
      // between-partial term of the merged centred sum of squares, about the
      // row mean (b holds the partials' own centred sums)
      const float mean = a / static_cast<float>(N);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = lane + 64 * j;
        if (s < S_st) {
          const float n = count_of(s, v2[j]);
          if (n > 0.f) {
            const float dm = v0[j] / n - mean;
            b += n * dm * dm;
          }
        }
      }
    }
  } else {
    // unrolled so that the partials' loads go out together (the sums keep their order)
#pragma unroll 8
    for (int s = lane; s < S_st; s += 64) {
      const float* m = mcol + s * sstr;
      a += m[0];
      b += m[1];
      if (ms == 4) {
        c += m[2];
        d += m[3];
      }
    }
    a = wave_sum(a);
    if (mode == kTauChan) {
      const float mean = a / static_cast<float>(N);
#pragma unroll 8
      for (int s = lane; s < S_st; s += 64) {
        const float n = count_of(s, ms >= 3 ? mcol[s * sstr + 2] : 0.f);
        if (n > 0.f) {
          const float dm = mcol[s * sstr] / n - mean;
          b += n * dm * dm;
        }
      }
    }
  }
  b = wave_sum(b);
  if (q.token_diag && ms == 4) {
    c = wave_sum(c);
    d = wave_sum(d);
  }
  TauRow r;
  const float fN = static_cast<float>(N);
  r.mean = a / fN;
  r.sd = (mode == kTauChan ? sqrtf(b / fN) : sqrtf(b / fN - __fmul_rn(r.mean, r.mean))) + 1e-8f;
  r.tv = r.mean + __fmul_rn(q.tau_off[t], r.sd);
  r.c = c;
  r.d = d;
  return r;
}

__device__ __attribute__((always_inline)) inline void tau_body(const TauParams& q, const int bid) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(bid) * 4 + (threadIdx.x >> 6);
  if (t >= q.T) return;
  const TauRow r = tau_row(q, t, lane);
  if (lane == 0) {
    q.tau[t] = r.tv;
    if (q.sstd) q.sstd[t] = r.sd;
    if (q.token_diag) {
      float* td = q.token_diag + t * SRW_TDIAG_COUNT;
      td[SRW_TDIAG_S_MEAN] = r.mean;
      td[SRW_TDIAG_S_STD] = r.sd;
      td[SRW_TDIAG_TAU] = r.tv;
      td[SRW_TDIAG_SUM_S3] = r.c;
      td[SRW_TDIAG_SUM_S4] = r.d;
    }
  }
}
__global__ __launch_bounds__(256) void srw_tau_kernel(TauParams q) { tau_body(q, blockIdx.x); }
__global__ __launch_bounds__(256) void srw_tau_batch_kernel(Batch<TauParams> b) {
  const int i = batch_index(b.start, b.n, blockIdx.x);
  tau_body(b.p[i], blockIdx.x - b.start[i]);
}

// ---------------------------------------------------------------------------
// finalize: reduce the N-splits, bf16-round each reference chunk's write GEMM,
// divide by den, round, scale.  One workgroup per row: the per-token partials
// are reduced once, then each thread sums its columns over the splits with
// eight independent loads in flight.
// ---------------------------------------------------------------------------

// The row's gate and intensity maxima for token_diag from its TP_SMAX
// partials' max m.  v4.1: m is the max score, and gate and intensity are
// non-decreasing in the score (v41:583, 536-537).  The v4.0.1 gate (den_gate):
// m is the max gate itself (v401:321), and there is no intensity.
__device__ __attribute__((always_inline)) inline void diag_maxima(const FinalParams& p, int64_t t, float m, float* td) {
  if (p.den_gate) {
    td[SRW_TDIAG_GATE_MAX] = m;
    td[SRW_TDIAG_INT_MAX] = 0.f;
    return;
  }
  const float tau_thr = p.tau[t] + p.gp.thr;
  const float tau_cut = tau_thr + p.gp.cut;
  const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(fmaf(m, p.exp_scale, -tau_thr * p.exp_scale)));
  const float imax = p.gp.eps + __builtin_amdgcn_fmed3f(m - tau_cut, 0.0f, p.gp.maxi);
  td[SRW_TDIAG_GATE_MAX] = act * imax;
  td[SRW_TDIAG_INT_MAX] = imax;
}

// NG: split groups per workgroup; VW: columns per thread (1, 2 or 4: 4-,
// 8- or 16-byte loads; the widest that leaves two workgroups per CU).  One workgroup per (row, block of 256 / NG
// x VW columns); thread (g, c) = (tid / CW, tid % CW) sums columns
// VW c .. VW c + VW - 1 of its block over splits s = g, g + NG, ... of each
// chunk with eight loads in flight; the NG group sums of a chunk combine in
// a fixed order, so the result is deterministic (and the same for either
// VW: each column keeps its order of additions).  Few splits per chunk
// (large T) use NG = 1, many (decode) NG = 16.
template <int NG, int VW>
__device__ __attribute__((always_inline)) inline void finalize_body(const FinalParams& p, const int bx, const int by) {
  constexpr int CW = 256 / NG;
  static_assert(VW == 1 || VW == 2 || VW == 4, "one, two or four columns per thread");
  typedef float vec_t __attribute__((ext_vector_type(VW)));
  __shared__ float red[3][4];
  __shared__ vec_t part[NG > 1 ? NG : 1][CW];
  const int64_t t = bx;
  const int tid = threadIdx.x;
  const int g = tid / CW, c = tid % CW;
  const int64_t stride = p.T * p.D;
  const int d = (by * CW + c) * VW;
  const bool dok = d < p.D;
  const vec_t* col = reinterpret_cast<const vec_t*>(p.out_part + t * p.D + (dok ? d : 0));
  const int64_t vstride = stride / VW;
  // many splits per chunk (decode): when one round of eight loads per thread
  // covers a chunk, the first chunk's loads go out before the per-token
  // partials are reduced and each next chunk's before the current one is
  // (the additions keep their order)
  const bool one_round = NG > 1 && p.spc <= 8 * NG;
  auto load_chunk = [&](int s0, vec_t (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int s = s0 + g + NG * j;
      v[j] = s < s0 + p.spc ? col[s * vstride] : vec_t{};
    }
  };
  vec_t cur[8];
  if (one_round) load_chunk(0, cur);
  float gs = 0.f, is = 0.f, na = 0.f;
  for (int s = tid; s < p.S_tok; s += 256) {
    const float* tp = p.tok_part + (static_cast<int64_t>(s) * p.T + t) * p.tps;
    gs += tp[0];
    is += tp[1];
    na += tp[2];
  }
  gs = wave_sum(gs);
  is = wave_sum(is);
  na = wave_sum(na);
  if ((tid & 63) == 0) {
    red[0][tid >> 6] = gs;
    red[1][tid >> 6] = is;
    red[2][tid >> 6] = na;
  }
  __syncthreads();
  const float G = red[0][0] + red[0][1] + red[0][2] + red[0][3];
  const float I = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  const float NA = red[2][0] + red[2][1] + red[2][2] + red[2][3];
  const float den = fmaxf(p.den_gate ? G : I, 1.0f);          // v41:584, v401:340
  vec_t raw = {};
  auto round_v = [](vec_t x) {
    vec_t r;
#pragma unroll
    for (int k = 0; k < VW; ++k) r[k] = round_bf16(x[k]);
    return r;
  };
  if (NG == 1 && p.spc == 1) {
    // one split per chunk: the chunks' loads go out eight at a time, the
    // rounded chunk results add in chunk order
    for (int s0 = 0; s0 < p.S; s0 += 8) {
      vec_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = s0 + j < p.S ? col[(s0 + j) * vstride] : vec_t{};
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < p.S) raw += round_v(v[j]);                  // bf16 dot output (v41:518)
    }
  }
  for (int s0 = 0; s0 < p.S && !(NG == 1 && p.spc == 1); s0 += p.spc) {  // one reference chunk
    vec_t acc[8] = {};
    if (one_round) {
      vec_t nxt[8] = {};
      if (s0 + p.spc < p.S) load_chunk(s0 + p.spc, nxt);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += cur[j];
#pragma unroll
      for (int j = 0; j < 8; ++j) cur[j] = nxt[j];
    } else {
      // rounds of eight splits per thread, all eight loads in flight at once
      // (predicated past the chunk's end)
      for (int s = s0 + g; s < s0 + p.spc; s += 8 * NG) {
        vec_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = s + NG * j < s0 + p.spc ? col[(s + NG * j) * vstride] : vec_t{};
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += v[j];
      }
    }
    const vec_t sum = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    if constexpr (NG == 1) {
      raw += round_v(sum);                                   // bf16 dot output (v41:518)
    } else {
      part[g][c] = sum;
      __syncthreads();
      if (g == 0) {
        vec_t q = part[0][c];
#pragma unroll
        for (int k = 1; k < NG; ++k) q += part[k][c];
        raw += round_v(q);                                   // bf16 dot output (v41:518)
      }
      __syncthreads();
    }
  }
  if (g == 0 && dok) {
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      const float o = round_bf16(raw[k] / den);             // v41:585-586
      p.out[t * p.D + d + k] = f32_to_bf16_bits(o * p.scale);
    }
  }
  if (by != 0) return;
  if (tid == 0) {
    if (p.gate_sum) p.gate_sum[t] = G;
    if (p.den) p.den[t] = den;
    if (p.n_active) p.n_active[t] = static_cast<int32_t>(NA);
  }
  if (p.token_diag && tid < 64) {
    // per-token diagnostics (v41:519-534); gate and intensity are
    // non-decreasing in the score, so their maxima follow from the max score
    float smax = -INFINITY, c[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = tid; s < p.S_tok; s += 64) {
      const float* tp = p.tok_part + (static_cast<int64_t>(s) * p.T + t) * p.tps;
      smax = fmaxf(smax, tp[TP_SMAX]);
#pragma unroll
      for (int k = 0; k < 6; ++k) c[k] += tp[TP_STRONG + k];
    }
    smax = wave_max(smax);
#pragma unroll
    for (int k = 0; k < 6; ++k) c[k] = wave_sum(c[k]);
    if (tid == 0) {
      float* td = p.token_diag + t * SRW_TDIAG_COUNT;
      diag_maxima(p, t, smax, td);
      td[SRW_TDIAG_INT_SUM] = I;
      td[SRW_TDIAG_N_STRONG] = c[0];
      td[SRW_TDIAG_N_BOUNDARY] = c[1];
      td[SRW_TDIAG_N_BAND075] = c[2];
      td[SRW_TDIAG_N_BAND030] = c[3];
      td[SRW_TDIAG_N_INT_CAP] = c[4];
      td[SRW_TDIAG_G_LOG_G] = c[5];
    }
  }
}
template <int NG, int VW = 1>
__global__ __launch_bounds__(256) void srw_finalize_kernel(FinalParams p) {
  finalize_body<NG, VW>(p, blockIdx.x, blockIdx.y);
}
template <int NG, int VW = 1>
__global__ __launch_bounds__(256) void srw_finalize_batch_kernel(Batch<FinalParams> b) {
  const int i = batch_index(b.start, b.n, blockIdx.x);
  finalize_body<NG, VW>(b.p[i], blockIdx.x - b.start[i], blockIdx.y);
}

// Few splits per chunk (spc < 16: prefill-sized T): one wave per row, lane l
// owning columns l + 64 j (coalesced 256-byte loads), four rows per
// workgroup.  Each chunk's splits are summed in the order of the NG = 1
// kernel above (eight accumulators, a fixed tree), so both give the same
// bits; the per-row partials and diagnostics are reduced across the wave.
template <int DC>  // d_model / 64
__device__ __attribute__((always_inline)) inline void finalize_rows_body(const FinalParams& p, const int bid) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(bid) * 4 + (threadIdx.x >> 6);
  if (t >= p.T) return;
  float gs = 0.f, is = 0.f, na = 0.f;
  for (int s = lane; s < p.S_tok; s += 64) {
    const float* tp = p.tok_part + (static_cast<int64_t>(s) * p.T + t) * p.tps;
    gs += tp[0];
    is += tp[1];
    na += tp[2];
  }
  gs = wave_sum(gs);
  is = wave_sum(is);
  na = wave_sum(na);
  const float den = fmaxf(p.den_gate ? gs : is, 1.0f);        // v41:584, v401:340
  const int64_t stride = p.T * p.D;
  // columns of element j of a lane: DC even, pairs (2 lane, 2 lane + 1) +
  // 128 (j / 2) read as 8-byte loads; DC odd, lane + 64 j.  The sum over the
  // splits runs in the same order for every column either way.
  constexpr bool PAIR = DC % 2 == 0;
  auto col_of = [&](int j) { return PAIR ? 2 * lane + (j & 1) + 128 * (j >> 1) : lane + 64 * j; };
  const float* row = p.out_part + t * p.D;
  float raw[DC];
#pragma unroll
  for (int j = 0; j < DC; ++j) raw[j] = 0.f;
  auto load_split = [&](int s, float (&v)[DC]) {
    const float* src = row + static_cast<int64_t>(s) * stride;
#pragma unroll
    for (int j = 0; j < DC; j += PAIR ? 2 : 1) {
      if constexpr (PAIR) {
        const float2 q = *reinterpret_cast<const float2*>(src + col_of(j));
        v[j] = q.x;
        v[j + 1] = q.y;
      } else {
        v[j] = src[col_of(j)];
      }
    }
  };
  for (int s0 = 0; s0 < p.S; s0 += p.spc) {                   // one reference chunk
    float acc[DC][8];
#pragma unroll
    for (int j = 0; j < DC; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[j][k] = 0.f;
    int s = s0;
    for (; s + 7 < s0 + p.spc; s += 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float v[DC];
        load_split(s + k, v);
#pragma unroll
        for (int j = 0; j < DC; ++j) acc[j][k] += v[j];
      }
    }
    for (; s < s0 + p.spc; ++s) {
      float v[DC];
      load_split(s, v);
#pragma unroll
      for (int j = 0; j < DC; ++j) acc[j][0] += v[j];
    }
#pragma unroll
    for (int j = 0; j < DC; ++j) {
      const float* a = acc[j];
      const float sum = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
      raw[j] += round_bf16(sum);                              // bf16 dot output (v41:518)
    }
  }
#pragma unroll
  for (int j = 0; j < DC; j += PAIR ? 2 : 1) {
    if constexpr (PAIR) {
      const uint32_t lo = f32_to_bf16_bits(round_bf16(raw[j] / den) * p.scale);       // v41:585-586
      const uint32_t hi = f32_to_bf16_bits(round_bf16(raw[j + 1] / den) * p.scale);
      *reinterpret_cast<uint32_t*>(p.out + t * p.D + col_of(j)) = lo | (hi << 16);
    } else {
      const float o = round_bf16(raw[j] / den);                 // v41:585-586
      p.out[t * p.D + col_of(j)] = f32_to_bf16_bits(o * p.scale);
    }
  }
  if (lane == 0) {
    if (p.gate_sum) p.gate_sum[t] = gs;
    if (p.den) p.den[t] = den;
    if (p.n_active) p.n_active[t] = static_cast<int32_t>(na);
  }
  if (p.token_diag) {
    float smax = -INFINITY, c[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = lane; s < p.S_tok; s += 64) {
      const float* tp = p.tok_part + (static_cast<int64_t>(s) * p.T + t) * p.tps;
      smax = fmaxf(smax, tp[TP_SMAX]);
#pragma unroll
      for (int k = 0; k < 6; ++k) c[k] += tp[TP_STRONG + k];
    }
    smax = wave_max(smax);
#pragma unroll
    for (int k = 0; k < 6; ++k) c[k] = wave_sum(c[k]);
    if (lane == 0) {
      float* td = p.token_diag + t * SRW_TDIAG_COUNT;
      diag_maxima(p, t, smax, td);
      td[SRW_TDIAG_INT_SUM] = is;
      td[SRW_TDIAG_N_STRONG] = c[0];
      td[SRW_TDIAG_N_BOUNDARY] = c[1];
      td[SRW_TDIAG_N_BAND075] = c[2];
      td[SRW_TDIAG_N_BAND030] = c[3];
      td[SRW_TDIAG_N_INT_CAP] = c[4];
      td[SRW_TDIAG_G_LOG_G] = c[5];
    }
  }
}

template <int DC>
__global__ __launch_bounds__(256) void srw_finalize_rows_kernel(FinalParams p) {
  finalize_rows_body<DC>(p, blockIdx.x);
}
template <int DC>
__global__ __launch_bounds__(256) void srw_finalize_rows_batch_kernel(Batch<FinalParams> b) {
  const int i = batch_index(b.start, b.n, blockIdx.x);
  finalize_rows_body<DC>(b.p[i], blockIdx.x - b.start[i]);
}

// ---------------------------------------------------------------------------
// unit diagnostics: unit_diag[u] = (sum of the unit's scores over all rows,
// its max gate) from the main kernel's per-32-row-block partials
// (v41:445-447, 543-552).  The gate is non-decreasing in the margin, so the
// max gate is the gate of the max margin (max of s - tau, minus thr).  A
// workgroup holds 64 units x 4 row slices; each slice sums its blocks in
// order, the slices combine in LDS in slice order: the result is the same on
// every call (the atomics it replaces summed in arrival order).
// ---------------------------------------------------------------------------
// gate_direct: the partials carry the max gate itself (the v4.0.1 gate, whose
// z scale differs per row), not the max margin.
__global__ __launch_bounds__(256) void srw_unit_diag_kernel(const float2* __restrict__ part, int64_t rows, int64_t N,
                                                            float* __restrict__ unit_diag, GateParams gp,
                                                            float exp_scale, int gate_direct) {
  __shared__ float2 red[4][64];
  const int ul = threadIdx.x & 63, slice = threadIdx.x >> 6;
  const int64_t u = static_cast<int64_t>(blockIdx.x) * 64 + ul;
  float su = 0.f, mx = -INFINITY;
  if (u < N) {
    int64_t r = slice;
    for (; r + 12 < rows; r += 16) {  // four blocks in flight per thread
      const float2 a = part[r * N + u], b = part[(r + 4) * N + u];
      const float2 c = part[(r + 8) * N + u], e = part[(r + 12) * N + u];
      su += a.x;
      su += b.x;
      su += c.x;
      su += e.x;
      mx = fmaxf(fmaxf(mx, fmaxf(a.y, b.y)), fmaxf(c.y, e.y));
    }
    for (; r < rows; r += 4) {
      const float2 a = part[r * N + u];
      su += a.x;
      mx = fmaxf(mx, a.y);
    }
  }
  red[slice][ul] = make_float2(su, mx);
  __syncthreads();
  if (slice == 0 && u < N) {
    float s = red[0][ul].x, m = red[0][ul].y;
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      s += red[q][ul].x;
      m = fmaxf(m, red[q][ul].y);
    }
    unit_diag[u * SRW_UDIAG_COUNT + SRW_UDIAG_SCORE_SUM] = s;
    unit_diag[u * SRW_UDIAG_COUNT + SRW_UDIAG_GATE_MAX] =
        !(m > -INFINITY) ? 0.f : (gate_direct ? m : gate_of_margin(m - gp.thr, gp, exp_scale));
  }
}

// ---------------------------------------------------------------------------
// decode: at most 128 virtual rows (T <= 128, or T <= 64 paired).  The pool is
// streamed once: one workgroup per N-split of at most four 32-unit tiles, so
// every CU holds one split's operands.  Wave w loads the E and R fragments of
// tile ta + w and the W^T fragments of its D / 4 output columns over all the
// split's tiles straight into registers -- every load of the workgroup, the
// rows' thresholds included, is issued before any arithmetic -- while X and
// H (per virtual row) arrive in LDS.  Then wave w runs the score and read
// GEMMs of its tile for all rows (rows = columns of the transposed GEMMs),
// the gate epilogue, and hands P to LDS (over X, after a barrier); finally
// each wave runs the write GEMM of its columns over the split's tiles.  The
// per-row sums of the four tiles are combined in LDS in wave order.
// ---------------------------------------------------------------------------
constexpr int kDecTiles = 4;    // tiles per split (one per wave)
constexpr int kDecMinTiles = 3; // the fewest per split the geometry aims for
constexpr int kDecMaxRows = 128;

template <int TB, int DB, int KH>
constexpr int decode_lds_bytes() {
  return TB * (DB * 2 + KH) * kFragBytes + 4 * TB * 32 * 3 * 4 + 4 * 4;  // + the sparse-skip tile masks
}

// NT: the most tiles a split holds (the W^T registers are sized for it; two
// at the small pools, whose splits hold one or two tiles).  GL: the v4.0.1
// GELU gate (p.sstd; the row sums carry z+ where v4.1 has the intensity).
// SP: sparse skip (SRW_FLAG_SPARSE_SKIP): X, H, E and tau are loaded first;
// each wave marks the units of its tile that pass for some row (v4.1:
// margin > 0; GELU: s > tau, i.e. gate > 0), the marks of the split's tiles
// meet in LDS, and only then go out the R rows of marked units (a lane's
// row) and the W^T fragments' halves holding a marked unit (8 units, two runs
// of 4 (unit_of_k), x 32 columns: 512 contiguous bytes).  An unmarked unit's R row is zero, so its
// x.r and P are zero: exact under the GELU gate (its gate is 0 there); under
// v4.1 its epsilon-sized gate times x.r is left out of out only -- the gate
// and intensity sums, den and the pass bits still come from its score.
template <int TB, int DB, int KH, int NT, bool GL = false, bool SP = false>
__device__ __attribute__((always_inline)) inline void decode_body(const MainParams& p, const int bid) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  constexpr int D = DB * 32, DR = KH * 16, KX = D / 16, NDB = DB / 4;
  constexpr int FX = TB * KX, FH = TB * KH;
  static_assert(DB % 4 == 0, "four waves split the output column blocks");
  static_assert(FX % 4 == 0 && FH % 4 == 0, "fragments split evenly over the waves");
  static_assert(NT >= 1 && NT <= kDecTiles, "one tile per wave at most");
  static_assert(FX >= NT * TB * 2, "P reuses the X region");
  char* const xl = lds;                          // X fragments, later P
  char* const hl = lds + FX * kFragBytes;        // H fragments
  float* const red = reinterpret_cast<float*>(hl + FH * kFragBytes);  // [wave][TB][32][3]
  uint32_t* const umask = reinterpret_cast<uint32_t*>(red + 4 * TB * 32 * 3);  // [wave]: marked units (SP)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, col = lane & 31;
  // workgroup = (split, row-block group): with rb > 1 (TB == 1) each
  // workgroup of a split takes one 32-row block, rows from row0
  const int split = bid / p.rb;
  const int64_t row0 = static_cast<int64_t>(bid % p.rb) * 32 * TB;
  int ta, tb;
  int64_t lo, hi;
  split_range(p.g, p.g.spc, split, ta, tb, lo, hi);
  const int64_t Tv = p.g.T, N = p.g.N;
  const int R = p.routes;

  // X and H fragments of this workgroup's 32-row blocks: fragment (block,
  // k-step) is one KB, lane l's 16 bytes at 16 l (rows past Tv repeat the last)
#pragma unroll
  for (int q = 0; q < FX / 4; ++q) {
    const int f = wave + 4 * q, blk = f / KX, ks = f % KX;
    int64_t v = row0 + 32 * blk + col;
    v = v < Tv ? v : Tv - 1;
    g2lds16(p.x + (v / R) * D + 16 * ks + 8 * half, xl + f * kFragBytes);
  }
#pragma unroll
  for (int q = 0; q < FH / 4; ++q) {
    const int f = wave + 4 * q, blk = f / KH, ks = f % KH;
    int64_t v = row0 + 32 * blk + col;
    v = v < Tv ? v : Tv - 1;
    g2lds16(p.h + v * DR + 16 * ks + 8 * half, hl + f * kFragBytes);
  }
  // this wave's tile and row blocks: with fewer than four tiles the waves of
  // a tile take its row blocks in turn (wpt waves per tile); a wave without
  // work reloads the split's last tile, unused
  const int ntl = tb - ta;
  const int wpt = ntl == 1 ? 4 : (ntl == 2 ? 2 : 1);
  const int wi = wave / wpt, wb = wave % wpt;
  const bool have = wi < ntl && wb < TB;
  const int mt = have ? ta + wi : tb - 1;
  int64_t ur = static_cast<int64_t>(mt) * kUnitTile + col;
  ur = ur < N ? ur : N - 1;
  u32x4_t ef[KH], rf[KX];
#pragma unroll
  for (int ks = 0; ks < KH; ++ks) ef[ks] = *reinterpret_cast<const u32x4_t*>(p.emb + ur * DR + 16 * ks + 8 * half);
  // the R row of unit col of this wave's tile, and the W^T fragments of
  // column blocks wave * NDB + c for the split's tiles (SP: of marked units
  // only, tmask[i] the marks of tile i)
  u32x4_t wf[NT][2][NDB];
  auto load_r = [&](const uint32_t* tmask) {
#pragma unroll
    for (int ks = 0; ks < KX; ++ks) {
      rf[ks] = u32x4_t{};
      if (!SP || ((tmask[wi < NT ? wi : 0] >> col) & 1u))
        rf[ks] = *reinterpret_cast<const u32x4_t*>(p.read + ur * D + 16 * ks + 8 * half);
    }
  };
  // (every slot is set: past the split's tiles without SP the last tile is
  // loaded again, with SP zeros, so that the write GEMM runs over all NT
  // slots with P zero there, without branches)
  auto load_w = [&](const uint32_t* tmask, int i_lo = 0, int i_hi = NT) {
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      if (i < i_lo || i >= i_hi) continue;
      const int64_t tile = ta + (i < ntl ? i : ntl - 1);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < NDB; ++c) {
          const int db = wave * NDB + c;
          wf[i][j][c] = u32x4_t{};
          // lane half h of k-step j holds units 16 j + 4 h + (0..3) and
          // 16 j + 8 + 4 h + (0..3) (unit_of_k)
          if (!SP || (i < ntl && (((tmask[i] >> (16 * j + 4 * half)) | (tmask[i] >> (16 * j + 8 + 4 * half))) & 0xFu)))
            wf[i][j][c] = *reinterpret_cast<const u32x4_t*>(p.wp + ((tile * DB + db) * 2 + j) * 512 + lane * 8);
        }
    }
  };
  if constexpr (!SP) load_r(nullptr);
  // the rows' thresholds (srw_tau_kernel, v41:461-464)
  float tau_b[TB], sstd_b[TB];
#pragma unroll
  for (int b = 0; b < TB; ++b) {
    const int64_t t = row0 + 32 * b + col;
    tau_b[b] = p.tau[t < Tv ? t : Tv - 1];
    sstd_b[b] = GL ? p.sstd[t < Tv ? t : Tv - 1] : 1.f;
  }
  wait_vm0();
  barrier_lds();
#pragma unroll
  for (int b = 0; b < TB; ++b) {
    if (GL) sstd_b[b] = 1.0f / sstd_b[b];  // its reciprocal
    // the GELU gate of _srw_inference compares with bf16(tau)
    if (GL && p.gl_raw_bf16) tau_b[b] = __uint_as_float(pack_bf16(0.0f, tau_b[b]));
  }
  if constexpr (SP) {
    // mark the tile's units that pass for some row of this wave's blocks
    uint32_t um = 0;
    if (have) {
      const int64_t ut = static_cast<int64_t>(mt) * kUnitTile;
#pragma unroll
      for (int b = 0; b < TB; ++b) {
        if (b % wpt != wb) continue;
        f32x16_t sacc = {};
#pragma unroll
        for (int ks = 0; ks < KH; ++ks)
          sacc = mfma(ef[ks], *reinterpret_cast<const u32x4_t*>(hl + (b * KH + ks) * kFragBytes + lane * 16), sacc);
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const uint32_t sp = pack_bf16(sacc[v], sacc[v + 1]);   // the bf16 scores the gate sees
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float sv = e ? hi_f32(sp) : lo_f32(sp);
            const bool pass = GL ? sv - tau_b[b] > 0.0f : (sv - tau_b[b]) - p.gp.thr > 0.0f;
            const int uo = unit_of_acc(v + e, half);
            const int64_t u = ut + uo;
            if (pass && u >= lo && u < hi) um |= 1u << uo;
          }
        }
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) um |= __shfl_xor(um, o);
    if (lane == 0) umask[wave] = um;
    __syncthreads();
    uint32_t tmask[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
      tmask[i] = 0u;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        if (w / wpt == i) tmask[i] |= umask[w];
    }
    load_r(tmask);
    load_w(tmask);
    wait_vm0();
  }

  // score and read GEMMs of this wave's tile for every row block, gate epilogue
  const GateParams gp = p.gp;
  const int64_t u0 = static_cast<int64_t>(mt) * kUnitTile;
  const bool shared_tile = (u0 < lo) || (u0 + kUnitTile > hi && hi < N);
  const bool full_tile = u0 >= lo && u0 + kUnitTile <= hi;
  uint32_t pk[TB][8];
  float gsum[TB], isum[TB];
  uint32_t nact[TB];
#pragma unroll
  for (int b = 0; b < TB; ++b) {
    gsum[b] = 0.f;
    isum[b] = 0.f;
    nact[b] = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) pk[b][q] = 0;
  }
  f32x16_t sacc[TB], racc[TB];
#pragma unroll
  for (int b = 0; b < TB; ++b) {
    sacc[b] = f32x16_t{};
    racc[b] = f32x16_t{};
  }
  if constexpr (SP) {
    // (W^T is in registers already: no room for fragment buffers)
    if (have) {
#pragma unroll
      for (int b = 0; b < TB; ++b) {
        if (b % wpt != wb) continue;
#pragma unroll
        for (int ks = 0; ks < KH; ++ks)
          sacc[b] = mfma(ef[ks], *reinterpret_cast<const u32x4_t*>(hl + (b * KH + ks) * kFragBytes + lane * 16), sacc[b]);
#pragma unroll
        for (int ks = 0; ks < KX; ++ks)
          racc[b] = mfma(rf[ks], *reinterpret_cast<const u32x4_t*>(xl + (b * KX + ks) * kFragBytes + lane * 16), racc[b]);
      }
    }
  } else {
    // the score GEMMs of every row block first; then the first half of the
    // W^T fragments goes out into the registers E held, streaming in under
    // the read GEMMs, and the second half after them, under the gate.  The
    // blocks' H and X fragments are read from LDS in groups ahead of their
    // MFMAs (scheduling barriers keep the reads ahead), so that the MFMAs
    // issue back to back instead of each waiting out one LDS read.
    if (have) {
#pragma unroll
      for (int b = 0; b < TB; ++b) {
        if (b % wpt != wb) continue;
        u32x4_t hq[KH];
#pragma unroll
        for (int ks = 0; ks < KH; ++ks) hq[ks] = *reinterpret_cast<const u32x4_t*>(hl + (b * KH + ks) * kFragBytes + lane * 16);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KH; ++ks) sacc[b] = mfma(ef[ks], hq[ks], sacc[b]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_w(nullptr, 0, NT / 2);
    __builtin_amdgcn_sched_barrier(0);
    if (have) {
#pragma unroll
      for (int b = 0; b < TB; ++b) {
        if (b % wpt != wb) continue;
        constexpr int G = KX % 8 == 0 ? 8 : KX;
        u32x4_t xq[2][G];
#pragma unroll
        for (int k = 0; k < G; ++k) xq[0][k] = *reinterpret_cast<const u32x4_t*>(xl + (b * KX + k) * kFragBytes + lane * 16);
#pragma unroll
        for (int g = 0; g < KX / G; ++g) {
          if (g + 1 < KX / G) {
#pragma unroll
            for (int k = 0; k < G; ++k)
              xq[(g + 1) & 1][k] = *reinterpret_cast<const u32x4_t*>(xl + (b * KX + (g + 1) * G + k) * kFragBytes + lane * 16);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int k = 0; k < G; ++k) racc[b] = mfma(rf[g * G + k], xq[g & 1][k], racc[b]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_w(nullptr, NT / 2, NT);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (have) {
#pragma unroll
    for (int b = 0; b < TB; ++b) {
      if (b % wpt != wb) continue;
      const int64_t t = row0 + 32 * b + col;
      const float tau = tau_b[b], istd = sstd_b[b];
      uint32_t bits = 0;
      // the bounds test per unit only in a tile the split shares or the pool ends in
      auto gate16 = [&](auto full_t) {
        constexpr bool FULL = decltype(full_t)::value;
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const uint32_t sp = pack_bf16(sacc[b][v], sacc[b][v + 1]);   // bf16 scores (v41:503)
          const uint32_t xp = pack_bf16(racc[b][v], racc[b][v + 1]);   // bf16 x.r (v41:517)
          float g2[2], in2[2];
          bool on2[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const float sv = e ? hi_f32(sp) : lo_f32(sp);
            const int64_t u = u0 + unit_of_acc(v + e, half);
            const bool ok = FULL || (u >= lo && u < hi);
            if constexpr (GL) {
              float zp;
              const float g = gelu_gate(sv, tau, istd, zp, p.gl_raw_bf16 != 0);
              g2[e] = ok ? g : 0.f;
              in2[e] = ok ? zp : 0.f;
              on2[e] = ok && zp > 0.0f;
            } else {
              const float raw = sv - tau;
              const float margin = raw - gp.thr;
              const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(margin * p.exp_scale));
              const float am = fmaxf(margin - gp.cut, 0.0f);
              g2[e] = ok ? act * (gp.eps + fminf(am, gp.maxi)) : 0.f;
              in2[e] = ok ? gp.eps + fminf(am, gp.maxi) : 0.f;
              on2[e] = ok && act > 0.5f;
            }
          }
          gsum[b] += g2[0];
          gsum[b] += g2[1];
          isum[b] += in2[0];
          isum[b] += in2[1];
          bits = (bits << 2) | (on2[0] ? 2u : 0u) | (on2[1] ? 1u : 0u);
          const uint32_t gq = pack_bf16(g2[0], g2[1]);             // gate_bf (v41:516)
          pk[b][v >> 1] = pack_bf16(lo_f32(gq) * lo_f32(xp), hi_f32(gq) * hi_f32(xp));  // (v41:518)
        }
      };
      if (full_tile) gate16(std::true_type{});
      else gate16(std::false_type{});
      // pass bits of (row, tile): element v at bit unit_of_acc(v, half)
      const uint32_t br = __builtin_bitreverse32(bits) >> 16;
      uint32_t m = (br & 0xFu) | ((br & 0xF0u) << 4) | ((br & 0xF00u) << 8) | ((br & 0xF000u) << 12);
      m <<= 4 * half;
      nact[b] = __builtin_popcount(m);
      m |= __shfl_xor(m, 32);
      if (p.mask32 && half == 0 && t < Tv) {
        uint32_t* dst = p.mask32 + t * p.mask_words32 + mt;
        if (shared_tile) atomicOr(dst, m);
        else *dst = m;
      }
    }
  }
  // per-row sums of each (tile, row block) this wave computed, into LDS
  if (have) {
#pragma unroll
    for (int b = 0; b < TB; ++b) {
      if (b % wpt != wb) continue;
      const float g = gsum[b] + __shfl_xor(gsum[b], 32);
      const float in = isum[b] + __shfl_xor(isum[b], 32);
      const uint32_t na = nact[b] + __shfl_xor(nact[b], 32);
      if (half == 0) {
        float* r = red + ((wi * TB + b) * 32 + col) * 3;
        r[0] = g;
        r[1] = in;
        r[2] = static_cast<float>(na);
      }
    }
  }
  barrier_lds();  // every wave is done reading X (the W^T loads stay in flight)
  // P of (tile wi, block b, k-step j) over X: lane l's 16 bytes at 16 l
  if (have) {
#pragma unroll
    for (int b = 0; b < TB; ++b) {
      if (b % wpt != wb) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        *reinterpret_cast<u32x4_t*>(xl + ((wi * TB + b) * 2 + j) * kFragBytes + lane * 16) =
            u32x4_t{pk[b][4 * j], pk[b][4 * j + 1], pk[b][4 * j + 2], pk[b][4 * j + 3]};
    }
  }
  barrier_lds();

  // write GEMM: OUT[rows x 32 (wave NDB + c) .. ] over the split's tiles, one
  // column block at a time, each stored while the next one runs
  u32x4_t pf[NT][2][TB];  // zero past the split's tiles
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int b = 0; b < TB; ++b) {
        pf[i][j][b] = u32x4_t{};
        if (i < ntl) pf[i][j][b] = *reinterpret_cast<const u32x4_t*>(xl + ((i * TB + b) * 2 + j) * kFragBytes + lane * 16);
      }
  float* op = p.out_part + static_cast<int64_t>(split) * Tv * D;
  // the lane's element (b, v) of column block c at lrow + (32 b + 8 (v / 4) +
  // v % 4) D + 32 c: compile-time offsets from one per-lane base
  float* lrow = op + (row0 + 4 * half) * D + 32 * wave * NDB + col;
#pragma unroll
  for (int c = 0; c < NDB; ++c) {
    f32x16_t oacc[TB];
#pragma unroll
    for (int b = 0; b < TB; ++b) oacc[b] = f32x16_t{};
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int b = 0; b < TB; ++b) oacc[b] = mfma(pf[i][j][b], wf[i][j][c], oacc[b]);
    // non-temporal stores: the partials go out to memory while the kernel
    // runs instead of as dirty L2 lines written back at its end (the Know
    // call's decode kernel 19.0 -> 17.4 us; the finalize then reads them from
    // memory, 6.1 -> 7.3 us; the decode step 0.727 -> 0.721 ms)
    if (row0 + 32 * TB <= Tv) {
#pragma unroll
      for (int b = 0; b < TB; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          __builtin_nontemporal_store(oacc[b][v], lrow + (32 * b + 8 * (v >> 2) + (v & 3)) * D + 32 * c);
    } else {
#pragma unroll
      for (int b = 0; b < TB; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t t = row0 + 32 * b + unit_of_acc(v, half);
          if (t < Tv) __builtin_nontemporal_store(oacc[b][v], lrow + (32 * b + 8 * (v >> 2) + (v & 3)) * D + 32 * c);
        }
    }
  }
  // per-row partials of the split: its tiles in order
  for (int r = threadIdx.x; r < TB * 32 && row0 + r < Tv; r += 256) {
    const int b = r / 32, c = r % 32;
    float acc[3] = {0.f, 0.f, 0.f};
    for (int i = 0; i < ntl; ++i)
#pragma unroll
      for (int k = 0; k < 3; ++k) acc[k] += red[((i * TB + b) * 32 + c) * 3 + k];
    float* tp = p.tok_part + (static_cast<int64_t>(split) * Tv + row0 + r) * 4;
    tp[0] = acc[0];
    tp[1] = acc[1];
    tp[2] = acc[2];
  }
}
// two waves per SIMD (two workgroups per CU) where the registers allow: the
// small pools' splits of one or two tiles
template <int TB, int DB, int KH, int NT = kDecTiles, bool GL = false, bool SP = false>
__global__ __launch_bounds__(256, NT <= 2 ? 2 : 1) void srw_decode_kernel(MainParams p) {
  decode_body<TB, DB, KH, NT, GL, SP>(p, blockIdx.x);
}
template <int TB, int DB, int KH, int NT = kDecTiles>
__global__ __launch_bounds__(256, NT <= 2 ? 2 : 1) void srw_decode_batch_kernel(Batch<MainParams> b) {
  const int i = batch_index(b.start, b.n, blockIdx.x);
  decode_body<TB, DB, KH, NT>(b.p[i], blockIdx.x - b.start[i]);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct Kernels {
  void (*stats)(StatsParams);
  void (*stats_chan)(StatsParams);  // the centred moments (kStatsChan), one pass
  void (*main)(MainParams);
  int main_threads;
  int main_lds;  // bytes
};

// WS: the warp-specialised main kernel (when both roles fit 256 registers);
// DG: with training diagnostics (warp-specialised kernels only)
// Token blocks per wave of the moments kernel.  Two (each E fragment feeding
// two MFMAs, half the E traffic per token) measured slower at the Know pool
// (0.431 against 0.402 ms per step): with x for 64 rows in registers one
// wave per SIMD remains, and the tile loop's waits are no longer hidden.
constexpr int kStatsTBW = 1;
template <int DB, int KH, bool HX, bool WS>
Kernels kernels_of(bool dg, bool gl = false) {
  if constexpr (WS) {
    constexpr int lds = (2 * (KH + 2 * DB) + 2 * 2 * DB + 16) * kFragBytes;  // 2 E/R, 2 W^T, S
    if (dg && gl)
      return Kernels{srw_stats_kernel<KH, kStatsDiag, 1>, srw_stats_kernel<KH, kStatsChan, 1>,
                     srw_main_ws_kernel<DB, KH, HX, true, true>, kWsThreads, lds};
    if (dg)
      return Kernels{srw_stats_kernel<KH, kStatsDiag, 1>, srw_stats_kernel<KH, kStatsChan, 1>,
                     srw_main_ws_kernel<DB, KH, HX, true>, kWsThreads, lds};
    if (gl)
      return Kernels{srw_stats_kernel<KH, kStatsPlain, kStatsTBW>, srw_stats_kernel<KH, kStatsChan, 1>,
                     srw_main_ws_kernel<DB, KH, HX, false, true>, kWsThreads, lds};
    return Kernels{srw_stats_kernel<KH, kStatsPlain, kStatsTBW>, srw_stats_kernel<KH, kStatsChan, 1>,
                   srw_main_ws_kernel<DB, KH, HX, false>, kWsThreads, lds};
  } else {
    return Kernels{srw_stats_kernel<KH, kStatsPlain, kStatsTBW>, srw_stats_kernel<KH, kStatsChan, 1>,
                   srw_main_kernel<DB, KH, HX>, kThreads, 2 * (KH + 2 * DB + 2 * DB) * kFragBytes};
  }
}

// Instantiated shapes (d_model, d_route); for d_route == d_model there is a
// variant whose score operand is the x registers themselves (h aliases x).
// gl: the v4.0.1 GELU gate (warp-specialised kernels).
bool pick(int64_t D, int64_t dr, bool hx, bool dg, Kernels* k, bool gl = false) {
  if (hx && D == dr) {
    if (D == 384) { *k = kernels_of<12, 24, true, true>(dg, gl); return true; }
    if (D == 128) { *k = kernels_of<4, 8, true, true>(dg, gl); return true; }
    if (D == 64) { *k = kernels_of<2, 4, true, true>(dg, gl); return true; }
  }
  if (D == 384 && dr == 384) {
    // the pipelined single-role kernel has no diagnostics or GELU variant
    if (dg || gl) return false;
    *k = kernels_of<12, 24, false, false>(false);
    return true;
  }
  if (D == 384 && dr == 128) { *k = kernels_of<12, 8, false, true>(dg, gl); return true; }
  if (D == 128 && dr == 128) { *k = kernels_of<4, 8, false, true>(dg, gl); return true; }
  if (D == 128 && dr == 64) { *k = kernels_of<4, 4, false, true>(dg, gl); return true; }
  if (D == 64 && dr == 64) { *k = kernels_of<2, 4, false, true>(dg, gl); return true; }
  if (D == 64 && dr == 32) { *k = kernels_of<2, 2, false, true>(dg, gl); return true; }
  return false;
}

bool with_diag(const srw_desc_t& d) { return (d.flags & SRW_FLAG_DIAG) != 0; }

// The decode kernel serves calls of at most 128 virtual rows without
// diagnostics, for the (d_model, d_route) pairs below.
bool decode_applies(const srw_desc_t& d) {
  const int64_t Tv = d.T * d.n_routes;
  if (with_diag(d) || Tv < 1 || Tv > kDecMaxRows) return false;
  return (d.d_model == 384 && d.d_route == 128) || (d.d_model == 128 && (d.d_route == 128 || d.d_route == 64));
}

typedef void (*MainFn)(MainParams);
template <int DB, int KH, bool GL, bool SP>
void decode_for_rows(int64_t Tv, int nt, MainFn* fn, int* lds) {
  if (Tv <= 32 && nt <= 2) {
    *fn = srw_decode_kernel<1, DB, KH, 2, GL, SP>;
    *lds = decode_lds_bytes<1, DB, KH>();
  } else if (Tv <= 32) {
    *fn = srw_decode_kernel<1, DB, KH, kDecTiles, GL, SP>;
    *lds = decode_lds_bytes<1, DB, KH>();
  } else if (Tv <= 64) {
    *fn = srw_decode_kernel<2, DB, KH, kDecTiles, GL, SP>;
    *lds = decode_lds_bytes<2, DB, KH>();
  } else {
    *fn = srw_decode_kernel<4, DB, KH, kDecTiles, GL, SP>;
    *lds = decode_lds_bytes<4, DB, KH>();
  }
}
template <bool GL, bool SP>
bool pick_decode_t(int64_t Tv, int D, int dr, int nt, MainFn* fn, int* lds) {
  if (D == 384 && dr == 128) {
    decode_for_rows<12, 8, GL, SP>(Tv, nt, fn, lds);
    return true;
  }
  if (D == 128 && dr == 128) {
    decode_for_rows<4, 8, GL, SP>(Tv, nt, fn, lds);
    return true;
  }
  if (D == 128 && dr == 64) {
    decode_for_rows<4, 4, GL, SP>(Tv, nt, fn, lds);
    return true;
  }
  return false;
}
// nt: the most tiles a split of the call holds (decode_max_tiles); gl: the
// v4.0.1 GELU gate; sp: sparse skip
bool pick_decode(int64_t Tv, int D, int dr, int nt, MainFn* fn, int* lds, bool gl = false, bool sp = false) {
  if (sp) return gl ? pick_decode_t<true, true>(Tv, D, dr, nt, fn, lds) : pick_decode_t<false, true>(Tv, D, dr, nt, fn, lds);
  return gl ? pick_decode_t<true, false>(Tv, D, dr, nt, fn, lds) : pick_decode_t<false, false>(Tv, D, dr, nt, fn, lds);
}
typedef void (*MainBatchFn)(Batch<MainParams>);
template <int DB, int KH>
MainBatchFn decode_batch_for(MainFn fn) {
  if (fn == srw_decode_kernel<1, DB, KH, 2>) return srw_decode_batch_kernel<1, DB, KH, 2>;
  if (fn == srw_decode_kernel<1, DB, KH>) return srw_decode_batch_kernel<1, DB, KH>;
  if (fn == srw_decode_kernel<2, DB, KH>) return srw_decode_batch_kernel<2, DB, KH>;
  if (fn == srw_decode_kernel<4, DB, KH>) return srw_decode_batch_kernel<4, DB, KH>;
  return nullptr;
}
// the batch twin of a decode kernel pick_decode returned
MainBatchFn decode_batch_of(MainFn fn) {
  if (MainBatchFn b = decode_batch_for<12, 8>(fn)) return b;
  if (MainBatchFn b = decode_batch_for<4, 8>(fn)) return b;
  return decode_batch_for<4, 4>(fn);
}
int mom_stride(const srw_desc_t& d) {
  if (d.stats_mode == SRW_STATS_CENTERED) return 3;  // kStatsChan: sum, M2, count
  return with_diag(d) && d.stats_mode == SRW_STATS_ONEPASS ? 4 : 2;
}
int tok_part_stride(const srw_desc_t& d) { return with_diag(d) ? kTokPartDiag : 4; }

Geometry geometry(const srw_desc_t& d, int64_t chunk) {
  Geometry g{};
  g.T = d.T * d.n_routes;  // virtual tokens (token, route)
  g.N = d.n_units;
  g.cs = chunk > 0 && chunk < d.n_units ? chunk : d.n_units;
  g.nc = static_cast<int>((g.N + g.cs - 1) / g.cs);
  g.TT = static_cast<int>((g.T + kTokTile - 1) / kTokTile);
  g.ntiles = static_cast<int>((g.N + kUnitTile - 1) / kUnitTile);
  // every split needs >= 1 tile: a chunk of L units spans >= L / 32 tiles
  const int64_t last = g.N - (g.nc - 1) * g.cs;
  const int64_t min_tiles = (last < g.cs ? last : g.cs) / kUnitTile;
  int spc = static_cast<int>((kTargetBlocks + g.TT * g.nc - 1) / (g.TT * g.nc));
  if (spc < 1) spc = 1;
  if (spc > min_tiles) spc = static_cast<int>(min_tiles > 0 ? min_tiles : 1);
  if (decode_applies(d)) {
    // decode: splits of kDecMinTiles .. kDecTiles tiles, as few as fill the
    // CUs.  Small pools take more tiles per split than filling the CUs asks
    // for: every
    // split writes fp32 partials for all its rows (rows x d_model x 4 bytes,
    // more than the split's share of the pool when it holds one tile), so
    // fewer, longer splits win there -- at the 40M decode step the QK and V
    // calls (50 and 82 tiles, 128 and 64 rows) wrote 18 MB of partials for
    // 7.5 MB of pool with one tile per split; with three, 0.818 -> 0.728 ms
    // per step
    int64_t tpw = (g.ntiles + kTargetBlocks - 1) / kTargetBlocks;
    tpw = tpw < kDecMinTiles ? kDecMinTiles : (tpw > kDecTiles ? kDecTiles : tpw);
    int64_t nt_max = 0;
    for (int c = 0; c < g.nc; ++c) {
      const int64_t c_lo = c * g.cs, c_hi = (c + 1) * g.cs < g.N ? (c + 1) * g.cs : g.N;
      const int64_t nt = (c_hi + kUnitTile - 1) / kUnitTile - c_lo / kUnitTile;
      nt_max = nt > nt_max ? nt : nt_max;
    }
    const int64_t sd = (nt_max + tpw - 1) / tpw;
    const int64_t mt = min_tiles > 0 ? min_tiles : 1;
    spc = static_cast<int>(sd < mt ? sd : mt);
  }
  g.spc = spc;
  g.S = g.nc * spc;
  // the moments kernel: token tiles of 128 TBW rows; with one block per wave
  // two workgroups share a CU, with two (the registers of 64 rows) one does
  const int tbw = with_diag(d) ? 1 : kStatsTBW;
  g.TT_st = static_cast<int>((g.T + kTokTile * tbw - 1) / (kTokTile * tbw));
  const int64_t st_blocks = tbw == 1 ? 2 * kTargetBlocks : kTargetBlocks;
  int spc_st = static_cast<int>((st_blocks + g.TT_st * g.nc - 1) / (g.TT_st * g.nc));
  if (decode_applies(d)) spc_st = spc;  // one row tile: fewer, longer moment splits (fewer partials per row)
  if (spc_st < 1) spc_st = 1;
  if (spc_st > min_tiles) spc_st = static_cast<int>(min_tiles > 0 ? min_tiles : 1);
  g.spc_st = spc_st;
  g.S_st = g.nc * spc_st;
  if (d.stats_mode == SRW_STATS_GRAM) g.S_st = gram_moment_parts(d.d_route);  // moments from the Gram kernels
  return g;
}

// The most tiles a split holds when every split of the decode kernel holds
// 1 .. kDecTiles of them, else 0.
int decode_max_tiles(const Geometry& g) {
  int most = 0;
  for (int sp = 0; sp < g.S; ++sp) {
    int ta, tb;
    int64_t lo, hi;
    split_range(g, g.spc, sp, ta, tb, lo, hi);
    if (tb <= ta || tb - ta > kDecTiles) return 0;
    most = tb - ta > most ? tb - ta : most;
  }
  return most;
}
bool decode_splits_fit(const Geometry& g) { return decode_max_tiles(g) > 0; }

// The scores-streaming main kernel serves calls without diagnostics whose
// moments come from the moments kernel (one-pass or centred statistics; the
// Gram statistics compute no scores), that do not take the decode kernel, and
// whose score GEMM is as wide as the read GEMM (d_route >= d_model).  The
// score buffer costs 4 bytes of HBM traffic per (row, unit) whatever d_route
// is, while the recompute it saves is a d_route / (d_route + 2 d_model) share
// of the main kernel's MFMAs: at d_route = d_model = 384 (Know pool, T =
// 4096) streaming took the moments + main kernels from 307 to 278 us, at
// d_route = 128 (the model's pools, T = 16 384) from 394 to 416 us.
bool ss_applies(const srw_desc_t& d, const Geometry& g) {
  if (d.stats_mode == SRW_STATS_GRAM || d.gate != SRW_GATE_V41) return false;
  if (d.d_model != 384 && d.d_model != 128 && d.d_model != 64) return false;
  if (d.d_route < d.d_model) return false;
  if (decode_applies(d) && decode_splits_fit(g)) return false;
  return g.TT_st == g.TT;  // the moments kernel's 128-row token tiles are the main kernel's
}
// dg: with training diagnostics
bool pick_ss(int64_t D, MainFn* fn, int* lds, bool dg = false) {
  if (D == 384) {
    *fn = dg ? srw_main_ss_kernel<12, true> : srw_main_ss_kernel<12>;
    *lds = dg ? ss_lds_bytes<12, true>() : ss_lds_bytes<12>();
    return true;
  }
  if (D == 128) {
    *fn = dg ? srw_main_ss_kernel<4, true> : srw_main_ss_kernel<4>;
    *lds = dg ? ss_lds_bytes<4, true>() : ss_lds_bytes<4>();
    return true;
  }
  if (D == 64) {
    *fn = dg ? srw_main_ss_kernel<2, true> : srw_main_ss_kernel<2>;
    *lds = dg ? ss_lds_bytes<2, true>() : ss_lds_bytes<2>();
    return true;
  }
  return false;
}

struct WsLayout {
  size_t wp, mom, tau, gram, out_part, tok_part, scores, rn, wn, sstd, upart, total;
};

size_t al(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

WsLayout ws_layout(const srw_desc_t& d, const Geometry& g) {
  WsLayout w{};
  size_t off = 0;
  w.wp = off;
  off += al(static_cast<size_t>(g.ntiles) * kUnitTile * d.d_model * 2);
  w.mom = off;
  off += al(static_cast<size_t>(g.S_st) * g.T * mom_stride(d) * 4);
  w.tau = off;
  off += al(static_cast<size_t>(g.T) * 4);
  w.gram = off;
  if (d.stats_mode == SRW_STATS_GRAM) off += al(gram_workspace_bytes(d.n_units, d.d_route));
  w.out_part = off;
  off += al(static_cast<size_t>(g.S) * g.T * d.d_model * 4);
  w.tok_part = off;
  off += al(static_cast<size_t>(g.S) * g.T * tok_part_stride(d) * 4);
  w.scores = off;
  if (ss_applies(d, g)) off += al(static_cast<size_t>(g.TT) * g.ntiles * kScoreTileBytes);
  // the v4.0.1 gate: forward-normalised read and write rows, the rows' s_std
  w.rn = w.wn = w.sstd = off;
  if (d.gate == SRW_GATE_GELU_V401) {
    const size_t rows = al(static_cast<size_t>(d.n_units) * d.d_model * 2);
    w.wn = w.rn + rows;
    w.sstd = w.wn + rows;
    off = w.sstd + al(static_cast<size_t>(g.T) * 4);
  }
  // diagnostics: the unit statistics per 32-row block (MainParams::unit_part)
  w.upart = off;
  if (with_diag(d)) off += al(static_cast<size_t>((g.T + 31) / 32) * d.n_units * sizeof(float2));
  w.total = off;
  return w;
}

int64_t chunk_of(const srw_desc_t& d) {
  return d.chunk_size > 0 && d.chunk_size < d.n_units ? d.chunk_size : d.n_units;
}

}  // namespace

hipError_t pack_unit_major(const uint16_t* src, uint16_t* dst, int64_t N, int D, hipStream_t s) {
  const int64_t ntiles = (N + kUnitTile - 1) / kUnitTile;
  const int64_t rows = ntiles * 2 * (D / 32) * 64;
  int64_t blocks = (rows + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(pack_w_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, src, dst, N, D, rows);
  return hipGetLastError();
}

// Row-major bf16 GEMM on the moments kernel's tile loop: 128-row token tiles,
// ceil(N / 32) unit tiles split over about two workgroups per CU.
static Geometry rows_geometry(int64_t rows, int64_t n) {
  Geometry g{};
  g.T = rows;
  g.N = n;
  g.cs = n;
  g.nc = 1;
  g.ntiles = static_cast<int>((n + kUnitTile - 1) / kUnitTile);
  g.TT_st = static_cast<int>((rows + kTokTile - 1) / kTokTile);
  int spc = static_cast<int>((2 * kTargetBlocks + g.TT_st - 1) / g.TT_st);
  spc = spc < 1 ? 1 : (spc > g.ntiles ? g.ntiles : spc);
  g.spc_st = g.S_st = g.spc = g.S = spc;
  g.TT = g.TT_st;
  return g;
}

bool rows_gemm_supports(int64_t k) { return k == 384 || k == 128 || k == 64 || k == 32; }

int rows_gemm_splits(int64_t rows, int64_t n) { return rows > 0 && n > 0 ? rows_geometry(rows, n).S_st : 1; }

hipError_t rows_gemm(const uint16_t* a, int64_t rows, const uint16_t* b, int64_t n, int64_t k, uint16_t* out,
                     int64_t ld, float* mom, hipStream_t s) {
  if (rows <= 0 || n <= 0) return hipSuccess;
  if (!rows_gemm_supports(k) || ld % 8 != 0 || ld < (n + kUnitTile - 1) / kUnitTile * kUnitTile)
    return hipErrorInvalidValue;
  StatsParams sp{};
  sp.h = a;
  sp.emb = b;
  sp.mom = mom;
  sp.g = rows_geometry(rows, n);
  sp.s_out = out;
  sp.s_ld = ld;
  void (*fn)(StatsParams) = nullptr;
  switch (k) {
    case 384: fn = mom ? srw_stats_kernel<24, kStatsRows, 1> : srw_stats_kernel<24, kStatsRowsOnly, 1>; break;
    case 128: fn = mom ? srw_stats_kernel<8, kStatsRows, 1> : srw_stats_kernel<8, kStatsRowsOnly, 1>; break;
    case 64: fn = mom ? srw_stats_kernel<4, kStatsRows, 1> : srw_stats_kernel<4, kStatsRowsOnly, 1>; break;
    default: fn = mom ? srw_stats_kernel<2, kStatsRows, 1> : srw_stats_kernel<2, kStatsRowsOnly, 1>; break;
  }
  const size_t smem = static_cast<size_t>(2 * (k / 16)) * kFragBytes;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(smem));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(sp.g.TT_st * sp.g.S_st)), dim3(kThreads), smem, s, sp);
  return hipGetLastError();
}

int finalize_groups(int spc);
FinalParams final_params_of(const FinalizeArgs& f);

bool mfma_supports(const srw_desc_t& d, bool h_is_x) {
  if (d.dtype != SRW_BF16) return false;
  const bool gl = d.gate == SRW_GATE_GELU_V401;
  if (d.stats_mode != SRW_STATS_ONEPASS && d.stats_mode != SRW_STATS_CENTERED &&
      !(d.stats_mode == SRW_STATS_GRAM && gram_supports(d.d_route)))
    return false;
  if (d.stats_mode == SRW_STATS_CENTERED && with_diag(d)) return false;  // diagnostics: one-pass moments only
  if (d.n_routes != 1 && d.n_routes != 2) return false;  // paired QK: 2 rows per token
  // SRW_FLAG_SPARSE_SKIP: the decode kernel skips; the prefill kernels run dense
  if (d.flags & (SRW_FLAG_EMULATE | SRW_FLAG_NO_FAST)) return false;
  Kernels k;
  if (!pick(d.d_model, d.d_route, h_is_x, with_diag(d), &k, gl)) return false;
  // every reference chunk must hold at least one whole 32-unit tile
  const int64_t cs = chunk_of(d);
  const int64_t last = d.n_units - ((d.n_units + cs - 1) / cs - 1) * cs;
  return (last < cs ? last : cs) >= kUnitTile;
}

size_t mfma_workspace_bytes(const srw_desc_t& d) {
  const Geometry g = geometry(d, chunk_of(d));
  return ws_layout(d, g).total;
}

hipError_t mfma_forward(const LaunchArgs& a, const char** path_name) {
  const srw_desc_t& d = a.d;
  *path_name = "mfma_bf16";
  const bool hx = a.in.h == a.in.x;
  const bool dg = with_diag(d);
  const bool gl = d.gate == SRW_GATE_GELU_V401;
  Kernels k;
  if (!pick(d.d_model, d.d_route, hx, dg, &k, gl)) return hipErrorNotSupported;
  const Geometry g = geometry(d, a.chunk);
  const WsLayout L = ws_layout(d, g);
  if (a.ws_bytes < L.total) return hipErrorInvalidValue;
  uint16_t* wp = reinterpret_cast<uint16_t*>(a.ws + L.wp);
  float* mom = reinterpret_cast<float*>(a.ws + L.mom);
  float* out_part = reinterpret_cast<float*>(a.ws + L.out_part);
  float* tok_part = reinterpret_cast<float*>(a.ws + L.tok_part);
  uint16_t* scores = reinterpret_cast<uint16_t*>(a.ws + L.scores);
  MainFn ss_fn = nullptr;
  int ss_lds = 0;
  const bool ss = ss_applies(d, g) && pick_ss(d.d_model, &ss_fn, &ss_lds, dg);
  const int D = static_cast<int>(d.d_model);
  const int KH = static_cast<int>(d.d_route / 16);
  const int DB = D / 32;
  uint32_t* mask32 = reinterpret_cast<uint32_t*>(a.o.pass_mask);
  const int64_t mw32 = 2 * a.words;
  hipError_t e;

  float* tau = reinterpret_cast<float*>(a.ws + L.tau);
  const bool cached = (d.flags & SRW_FLAG_POOL_CACHED) != 0;
  float* token_diag = dg ? a.o.token_diag : nullptr;
  float* unit_diag = dg ? a.o.unit_diag : nullptr;
  float2* unit_part = unit_diag ? reinterpret_cast<float2*>(a.ws + L.upart) : nullptr;

  // the v4.0.1 gate reads forward-normalised rows (v401:300-301)
  const uint16_t* read_rows = static_cast<const uint16_t*>(a.in.read);
  const uint16_t* write_rows = static_cast<const uint16_t*>(a.in.write);
  float* sstd = gl ? reinterpret_cast<float*>(a.ws + L.sstd) : nullptr;
  if (gl) {
    uint16_t* rn = reinterpret_cast<uint16_t*>(a.ws + L.rn);
    uint16_t* wn = reinterpret_cast<uint16_t*>(a.ws + L.wn);
    if (!cached) {
      if ((e = normalize_rows_bf16(read_rows, rn, d.n_units, D, a.stream)) != hipSuccess) return e;
      if ((e = normalize_rows_bf16(write_rows, wn, d.n_units, D, a.stream)) != hipSuccess) return e;
    }
    read_rows = rn;
    write_rows = wn;
  }
  // decode-sized calls: the decode kernel (few splits -- small pools -- one
  // workgroup per (split, 32-row block), so that more CUs share the pool and
  // each loads only its rows' X and H)
  const int row_blocks = static_cast<int>((g.T + 31) / 32);
  const int rb = (row_blocks > 1 && static_cast<int64_t>(g.S) * row_blocks <= kTargetBlocks) ? row_blocks : 1;
  MainFn dec = nullptr;
  int dec_lds = 0;
  const bool decode = decode_applies(d) && decode_splits_fit(g) &&
                      pick_decode(rb > 1 ? 32 : g.T, D, static_cast<int>(d.d_route), decode_max_tiles(g), &dec, &dec_lds,
                                  gl, (d.flags & SRW_FLAG_SPARSE_SKIP) != 0);
  // pack W^T (kept in the workspace across calls that declare the pool cached)
  if (!cached) {
    const int64_t rows = static_cast<int64_t>(g.ntiles) * 2 * DB * 64;
    int64_t blocks = (rows + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(pack_w_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, a.stream, write_rows, wp,
                       d.n_units, D, rows);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // the finalize of the call
  FinalizeArgs f{};
  f.out_part = out_part;
  f.tok_part = tok_part;
  f.out = static_cast<uint16_t*>(a.o.out);
  f.gate_sum = a.o.gate_sum;
  f.den = a.o.den;
  f.n_active = a.o.n_active;
  f.T = g.T;
  f.D = D;
  f.S = g.S;
  f.spc = g.spc;
  f.S_tok = g.S;
  f.tps = tok_part_stride(d);
  f.scale = d.scale;
  f.tau = tau;
  f.token_diag = token_diag;
  f.gp = a.gp;
  f.exp_scale = -d.sharpness * 1.4426950408889634f;
  f.den_gate = gl ? 1 : 0;
  const unsigned grid = static_cast<unsigned>(g.TT * g.S);
  const unsigned grid_st = static_cast<unsigned>(g.TT_st * g.S_st);
  if (d.stats_mode == SRW_STATS_GRAM) {
    if ((e = gram_moments(static_cast<const uint16_t*>(a.in.emb), static_cast<const uint16_t*>(a.in.h), g.T,
                          d.n_units, d.d_route, mom, a.ws + L.gram, a.stream, mask32, mw32, g.cs, g.nc,
                          cached)) != hipSuccess)
      return e;
  } else {
    StatsParams sp{};
    sp.h = static_cast<const uint16_t*>(a.in.h);
    sp.emb = static_cast<const uint16_t*>(a.in.emb);
    sp.mom = mom;
    sp.mask32 = mask32;
    sp.mask_words32 = mw32;
    sp.g = g;
    sp.s_out = ss ? scores : nullptr;
    const size_t smem = static_cast<size_t>(2 * KH) * kFragBytes;
    // centred statistics: one pass (kStatsChan), the splits merged in srw_tau_kernel
    const auto stats_fn = d.stats_mode == SRW_STATS_CENTERED ? k.stats_chan : k.stats;
    if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(stats_fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 static_cast<int>(smem))) != hipSuccess)
      return e;
    hipLaunchKernelGGL(stats_fn, dim3(grid_st), dim3(kThreads), smem, a.stream, sp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  // tau per row from the moment partials
  if ((e = launch_tau(mom, a.in.tau_offset, tau, g.T, g.S_st, g.N, d.stats_mode == SRW_STATS_GRAM ? 2 : mom_stride(d),
                      token_diag, d.stats_mode == SRW_STATS_CENTERED ? kTauChan : kTauOnePass, a.stream, sstd)) !=
      hipSuccess)
    return e;
  // main
  {
    MainParams mp{};
    mp.x = static_cast<const uint16_t*>(a.in.x);
    mp.routes = d.n_routes;
    mp.h = static_cast<const uint16_t*>(a.in.h);
    mp.emb = static_cast<const uint16_t*>(a.in.emb);
    mp.read = read_rows;
    mp.wp = wp;
    mp.tau = tau;
    mp.sstd = sstd;
    mp.gl_raw_bf16 = gl && d.stats_mode == SRW_STATS_CENTERED;
    mp.out_part = out_part;
    mp.tok_part = tok_part;
    mp.unit_part = unit_part;
    mp.mask32 = mask32;
    mp.mask_words32 = mw32;
    mp.g = g;
    mp.gp = a.gp;
    mp.exp_scale = -d.sharpness * 1.4426950408889634f;
    mp.rb = rb;
    if (decode) {
      *path_name = (d.flags & SRW_FLAG_SPARSE_SKIP) ? "mfma_decode_sparse_bf16" : "mfma_decode_bf16";
      if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(dec), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   dec_lds)) != hipSuccess)
        return e;
      dominant_kernel_begin(a.stream);
      hipLaunchKernelGGL(dec, dim3(static_cast<unsigned>(g.S * mp.rb)), dim3(kThreads), static_cast<size_t>(dec_lds),
                         a.stream, mp);
      dominant_kernel_end(a.stream);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    } else {
      MainFn fn = k.main;
      int threads = k.main_threads, lds = k.main_lds;
      if (ss) {  // the moments kernel stored the scores
        *path_name = "mfma_ss_bf16";
        fn = ss_fn;
        threads = kWsThreads;
        lds = ss_lds;
        mp.s_in = scores;
      }
      if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   lds)) != hipSuccess)
        return e;
      dominant_kernel_begin(a.stream);
      hipLaunchKernelGGL(fn, dim3(grid), dim3(threads), static_cast<size_t>(lds), a.stream, mp);
      dominant_kernel_end(a.stream);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  // finalize
  if ((e = launch_finalize(f, a.stream)) != hipSuccess) return e;
  if (unit_part) {
    const int64_t rows = (g.T + 31) / 32;
    hipLaunchKernelGGL(srw_unit_diag_kernel, dim3(static_cast<unsigned>((d.n_units + 63) / 64)), dim3(256), 0,
                       a.stream, unit_part, rows, static_cast<int64_t>(d.n_units), unit_diag, a.gp, f.exp_scale,
                       gl ? 1 : 0);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_tau(const float* mom, const float* tau_off, float* tau, int64_t T, int S_st, int64_t N, int ms,
                      float* token_diag, int mode, hipStream_t s, float* sstd, int upp) {
  if (mode == kTauChan && upp <= 0 && ms < 3) return hipErrorInvalidValue;
  const TauParams q{mom, tau_off, tau, T, S_st, N, ms, token_diag, mode, sstd, upp};
  hipLaunchKernelGGL(srw_tau_kernel, dim3(static_cast<unsigned>((T + 3) / 4)), dim3(256), 0, s, q);
  return hipGetLastError();
}

// split groups per finalize workgroup from the splits per chunk
int finalize_groups(int spc) { return spc >= 32 ? 16 : (spc >= 16 ? 4 : 1); }
// columns per thread of srw_finalize_kernel: the widest loads (4, 2, 1
// floats) that D allows and that still leave at least two workgroups per CU
int finalize_width(int64_t rows, int D, int ng) {
  for (int vw = 4; vw > 1; vw /= 2) {
    const int cols = 256 / ng * vw;
    if (D % vw == 0 && rows * ((D + cols - 1) / cols) >= 2 * 256) return vw;
  }
  return 1;
}

FinalParams final_params_of(const FinalizeArgs& f) {
  FinalParams fp{};
  fp.out_part = f.out_part;
  fp.tok_part = f.tok_part;
  fp.out = f.out;
  fp.gate_sum = f.gate_sum;
  fp.den = f.den;
  fp.n_active = f.n_active;
  fp.T = f.T;
  fp.D = f.D;
  fp.S = f.S;
  fp.spc = f.spc;
  fp.S_tok = f.S_tok;
  fp.scale = f.scale;
  fp.tps = f.tps;
  fp.tau = f.tau;
  fp.token_diag = f.token_diag;
  fp.gp = f.gp;
  fp.exp_scale = f.exp_scale;
  fp.den_gate = f.den_gate;
  return fp;
}

hipError_t launch_finalize(const FinalizeArgs& f, hipStream_t s) {
  const FinalParams fp = final_params_of(f);
  const int ng = finalize_groups(f.spc);
  if (ng == 1 && (f.D == 64 || f.D == 128 || f.D == 384)) {
    const dim3 grid_r(static_cast<unsigned>((f.T + 3) / 4));
    if (f.D == 64) hipLaunchKernelGGL(srw_finalize_rows_kernel<1>, grid_r, dim3(256), 0, s, fp);
    else if (f.D == 128) hipLaunchKernelGGL(srw_finalize_rows_kernel<2>, grid_r, dim3(256), 0, s, fp);
    else hipLaunchKernelGGL(srw_finalize_rows_kernel<6>, grid_r, dim3(256), 0, s, fp);
    return hipGetLastError();
  }
  const int vw = finalize_width(f.T, f.D, ng);
  const int cols = 256 / ng * vw;  // per workgroup
  const dim3 grid_f(static_cast<unsigned>(f.T), static_cast<unsigned>((f.D + cols - 1) / cols));
  if (vw == 4) {
    if (ng == 16) hipLaunchKernelGGL((srw_finalize_kernel<16, 4>), grid_f, dim3(256), 0, s, fp);
    else if (ng == 4) hipLaunchKernelGGL((srw_finalize_kernel<4, 4>), grid_f, dim3(256), 0, s, fp);
    else hipLaunchKernelGGL((srw_finalize_kernel<1, 4>), grid_f, dim3(256), 0, s, fp);
  } else if (vw == 2) {
    if (ng == 16) hipLaunchKernelGGL((srw_finalize_kernel<16, 2>), grid_f, dim3(256), 0, s, fp);
    else if (ng == 4) hipLaunchKernelGGL((srw_finalize_kernel<4, 2>), grid_f, dim3(256), 0, s, fp);
    else hipLaunchKernelGGL((srw_finalize_kernel<1, 2>), grid_f, dim3(256), 0, s, fp);
  } else {
    if (ng == 16) hipLaunchKernelGGL(srw_finalize_kernel<16>, grid_f, dim3(256), 0, s, fp);
    else if (ng == 4) hipLaunchKernelGGL(srw_finalize_kernel<4>, grid_f, dim3(256), 0, s, fp);
    else hipLaunchKernelGGL(srw_finalize_kernel<1>, grid_f, dim3(256), 0, s, fp);
  }
  return hipGetLastError();
}

// The batch twin of a prefill main kernel (non-diagnostic instantiations).
MainBatchFn main_batch_of(MainFn fn) {
  if (fn == srw_main_ss_kernel<12>) return srw_main_ss_batch_kernel<12>;
  if (fn == srw_main_ss_kernel<4>) return srw_main_ss_batch_kernel<4>;
  if (fn == srw_main_ss_kernel<2>) return srw_main_ss_batch_kernel<2>;
  if (fn == srw_main_ws_kernel<12, 24, true, false>) return srw_main_ws_batch_kernel<12, 24, true>;
  if (fn == srw_main_ws_kernel<4, 8, true, false>) return srw_main_ws_batch_kernel<4, 8, true>;
  if (fn == srw_main_ws_kernel<2, 4, true, false>) return srw_main_ws_batch_kernel<2, 4, true>;
  if (fn == srw_main_ws_kernel<12, 8, false, false>) return srw_main_ws_batch_kernel<12, 8, false>;
  if (fn == srw_main_ws_kernel<4, 8, false, false>) return srw_main_ws_batch_kernel<4, 8, false>;
  if (fn == srw_main_ws_kernel<4, 4, false, false>) return srw_main_ws_batch_kernel<4, 4, false>;
  if (fn == srw_main_ws_kernel<2, 4, false, false>) return srw_main_ws_batch_kernel<2, 4, false>;
  if (fn == srw_main_ws_kernel<2, 2, false, false>) return srw_main_ws_batch_kernel<2, 2, false>;
  return nullptr;
}

// Several calls, one launch per stage (srw_forward_batch): every call must
// take the same main kernel instantiation -- all the decode kernel, or all
// the same prefill main kernel (scores streamed or recomputed) -- the same
// moments kernel and the same finalize grouping; otherwise nothing is
// launched and hipErrorNotSupported returned (the caller runs the calls one
// by one).  Each call keeps its own geometry, workspace and outputs, and its
// blocks run exactly the code of its own srw_forward: equal bits.
hipError_t mfma_forward_batch(const LaunchArgs* a, int n, const char** path_name) {
  if (n < 1 || n > kMaxBatch) return hipErrorNotSupported;
  Geometry g[kMaxBatch];
  WsLayout L[kMaxBatch];
  bool ss[kMaxBatch];
  int rb[kMaxBatch];
  MainFn main0 = nullptr;
  int lds0 = 0, threads0 = kThreads;
  const srw_desc_t& d0 = a[0].d;
  bool decode = false;
  for (int i = 0; i < n; ++i) {
    const srw_desc_t& d = a[i].d;
    // one call at a time: diagnostics, Gram statistics, the v4.0.1 gate, sparse skip
    if (with_diag(d) || d.stats_mode == SRW_STATS_GRAM || d.gate != SRW_GATE_V41 ||
        (d.flags & SRW_FLAG_SPARSE_SKIP))
      return hipErrorNotSupported;
    if (d.d_model != d0.d_model || d.d_route != d0.d_route || d.stats_mode != d0.stats_mode)
      return hipErrorNotSupported;
    g[i] = geometry(d, a[i].chunk);
    L[i] = ws_layout(d, g[i]);
    if (a[i].ws_bytes < L[i].total) return hipErrorInvalidValue;
    const bool dec_i = decode_applies(d) && decode_splits_fit(g[i]);
    if (i == 0) decode = dec_i;
    if (dec_i != decode) return hipErrorNotSupported;
    MainFn fn = nullptr;
    int lds = 0, threads = kThreads;
    ss[i] = false;
    rb[i] = 1;
    if (decode) {
      const int row_blocks = static_cast<int>((g[i].T + 31) / 32);
      rb[i] = (row_blocks > 1 && static_cast<int64_t>(g[i].S) * row_blocks <= kTargetBlocks) ? row_blocks : 1;
      if (!pick_decode(rb[i] > 1 ? 32 : g[i].T, static_cast<int>(d.d_model), static_cast<int>(d.d_route),
                       decode_max_tiles(g[i]), &fn, &lds))
        return hipErrorNotSupported;
    } else {
      Kernels k;
      if (!pick(d.d_model, d.d_route, a[i].in.h == a[i].in.x, false, &k)) return hipErrorNotSupported;
      MainFn ss_fn = nullptr;
      int ss_lds = 0;
      ss[i] = ss_applies(d, g[i]) && pick_ss(d.d_model, &ss_fn, &ss_lds);
      fn = ss[i] ? ss_fn : k.main;
      lds = ss[i] ? ss_lds : k.main_lds;
      threads = ss[i] ? kWsThreads : k.main_threads;
    }
    if (i > 0 && (fn != main0 || finalize_groups(g[i].spc) != finalize_groups(g[0].spc)))
      return hipErrorNotSupported;
    main0 = fn;
    lds0 = lds;
    threads0 = threads;
  }
  const MainBatchFn main_batch = decode ? decode_batch_of(main0) : main_batch_of(main0);
  if (!main_batch) return hipErrorNotSupported;
  const int ng = finalize_groups(g[0].spc);
  const bool rows_fin = ng == 1;  // the row-per-wave finalize, as launch_finalize picks it
  if (rows_fin && d0.d_model != 64 && d0.d_model != 128 && d0.d_model != 384) return hipErrorNotSupported;
  const int D = static_cast<int>(d0.d_model);
  const int KH = static_cast<int>(d0.d_route / 16);
  const bool centered = d0.stats_mode == SRW_STATS_CENTERED;
  void (*stats_plain)(Batch<StatsParams>) = nullptr;
  void (*stats_cent)(Batch<StatsParams>) = nullptr;
  switch (KH) {
    case 24: stats_plain = srw_stats_batch_kernel<24, kStatsPlain>; stats_cent = srw_stats_batch_kernel<24, kStatsChan>; break;
    case 8: stats_plain = srw_stats_batch_kernel<8, kStatsPlain>; stats_cent = srw_stats_batch_kernel<8, kStatsChan>; break;
    case 4: stats_plain = srw_stats_batch_kernel<4, kStatsPlain>; stats_cent = srw_stats_batch_kernel<4, kStatsChan>; break;
    case 2: stats_plain = srw_stats_batch_kernel<2, kStatsPlain>; stats_cent = srw_stats_batch_kernel<2, kStatsChan>; break;
    default: return hipErrorNotSupported;
  }
  const hipStream_t st = a[0].stream;
  hipError_t e;
  *path_name = decode ? "mfma_decode_batch_bf16" : "mfma_batch_bf16";

  // per call: pack W^T unless cached (its own launch)
  for (int i = 0; i < n; ++i) {
    if (a[i].d.flags & SRW_FLAG_POOL_CACHED) continue;
    if ((e = pack_unit_major(static_cast<const uint16_t*>(a[i].in.write), reinterpret_cast<uint16_t*>(a[i].ws + L[i].wp),
                             a[i].d.n_units, D, st)) != hipSuccess)
      return e;
  }
  // moments (centred statistics: kStatsChan, merged in the tau kernel)
  Batch<StatsParams> sb{};
  Batch<TauParams> tb{};
  sb.n = tb.n = n;
  for (int i = 0; i < n; ++i) {
    StatsParams& sp = sb.p[i];
    sp.h = static_cast<const uint16_t*>(a[i].in.h);
    sp.emb = static_cast<const uint16_t*>(a[i].in.emb);
    sp.mom = reinterpret_cast<float*>(a[i].ws + L[i].mom);
    sp.mask32 = reinterpret_cast<uint32_t*>(a[i].o.pass_mask);
    sp.mask_words32 = 2 * a[i].words;
    sp.g = g[i];
    sp.s_out = ss[i] ? reinterpret_cast<uint16_t*>(a[i].ws + L[i].scores) : nullptr;
    sb.start[i + 1] = sb.start[i] + g[i].TT_st * g[i].S_st;
    tb.p[i] = TauParams{sp.mom, a[i].in.tau_offset, reinterpret_cast<float*>(a[i].ws + L[i].tau), g[i].T,
                        g[i].S_st, g[i].N, centered ? 3 : 2, nullptr, centered ? kTauChan : kTauOnePass};
    tb.start[i + 1] = tb.start[i] + static_cast<int>((g[i].T + 3) / 4);
  }
  const size_t smem = static_cast<size_t>(2 * KH) * kFragBytes;
  for (auto fn : {stats_plain, stats_cent})
    if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 static_cast<int>(smem))) != hipSuccess)
      return e;
  hipLaunchKernelGGL(centered ? stats_cent : stats_plain, dim3(static_cast<unsigned>(sb.start[n])), dim3(kThreads),
                     smem, st, sb);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(srw_tau_batch_kernel, dim3(static_cast<unsigned>(tb.start[n])), dim3(256), 0, st, tb);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  // main (decode or prefill) kernel
  Batch<MainParams> mb{};
  mb.n = n;
  for (int i = 0; i < n; ++i) {
    const srw_desc_t& d = a[i].d;
    MainParams& mp = mb.p[i];
    mp.x = static_cast<const uint16_t*>(a[i].in.x);
    mp.routes = d.n_routes;
    mp.h = static_cast<const uint16_t*>(a[i].in.h);
    mp.emb = static_cast<const uint16_t*>(a[i].in.emb);
    mp.read = static_cast<const uint16_t*>(a[i].in.read);
    mp.wp = reinterpret_cast<const uint16_t*>(a[i].ws + L[i].wp);
    mp.tau = tb.p[i].tau;
    mp.out_part = reinterpret_cast<float*>(a[i].ws + L[i].out_part);
    mp.tok_part = reinterpret_cast<float*>(a[i].ws + L[i].tok_part);
    mp.mask32 = reinterpret_cast<uint32_t*>(a[i].o.pass_mask);
    mp.mask_words32 = 2 * a[i].words;
    mp.g = g[i];
    mp.gp = a[i].gp;
    mp.exp_scale = -d.sharpness * 1.4426950408889634f;
    mp.rb = rb[i];
    mp.s_in = ss[i] ? reinterpret_cast<const uint16_t*>(a[i].ws + L[i].scores) : nullptr;
    mb.start[i + 1] = mb.start[i] + (decode ? g[i].S * rb[i] : g[i].TT * g[i].S);
  }
  // the calls' finalize parameters
  Batch<FinalParams> fb{};
  fb.n = n;
  for (int i = 0; i < n; ++i) {
    const srw_desc_t& d = a[i].d;
    FinalizeArgs f{};
    f.out_part = mb.p[i].out_part;
    f.tok_part = mb.p[i].tok_part;
    f.out = static_cast<uint16_t*>(a[i].o.out);
    f.gate_sum = a[i].o.gate_sum;
    f.den = a[i].o.den;
    f.n_active = a[i].o.n_active;
    f.T = g[i].T;
    f.D = D;
    f.S = g[i].S;
    f.spc = g[i].spc;
    f.S_tok = g[i].S;
    f.tps = tok_part_stride(d);
    f.scale = d.scale;
    f.tau = tb.p[i].tau;
    f.token_diag = nullptr;
    f.gp = a[i].gp;
    f.exp_scale = -d.sharpness * 1.4426950408889634f;
    fb.p[i] = final_params_of(f);
    fb.start[i + 1] = fb.start[i] + static_cast<int>(rows_fin ? (g[i].T + 3) / 4 : g[i].T);
  }
  if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(main_batch), hipFuncAttributeMaxDynamicSharedMemorySize,
                               lds0)) != hipSuccess)
    return e;
  dominant_kernel_begin(st);
  hipLaunchKernelGGL(main_batch, dim3(static_cast<unsigned>(mb.start[n])), dim3(threads0),
                     static_cast<size_t>(lds0), st, mb);
  dominant_kernel_end(st);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  if (rows_fin) {
    const dim3 grid_r(static_cast<unsigned>(fb.start[n]));
    if (D == 64) hipLaunchKernelGGL(srw_finalize_rows_batch_kernel<1>, grid_r, dim3(256), 0, st, fb);
    else if (D == 128) hipLaunchKernelGGL(srw_finalize_rows_batch_kernel<2>, grid_r, dim3(256), 0, st, fb);
    else hipLaunchKernelGGL(srw_finalize_rows_batch_kernel<6>, grid_r, dim3(256), 0, st, fb);
    return hipGetLastError();
  }
  const int vw = finalize_width(fb.start[n], D, ng);
  const int cols = 256 / ng * vw;  // per workgroup
  const dim3 grid_f(static_cast<unsigned>(fb.start[n]), static_cast<unsigned>((D + cols - 1) / cols));
  if (vw == 4) {
    if (ng == 16) hipLaunchKernelGGL((srw_finalize_batch_kernel<16, 4>), grid_f, dim3(256), 0, st, fb);
    else hipLaunchKernelGGL((srw_finalize_batch_kernel<4, 4>), grid_f, dim3(256), 0, st, fb);
  } else if (vw == 2) {
    if (ng == 16) hipLaunchKernelGGL((srw_finalize_batch_kernel<16, 2>), grid_f, dim3(256), 0, st, fb);
    else hipLaunchKernelGGL((srw_finalize_batch_kernel<4, 2>), grid_f, dim3(256), 0, st, fb);
  } else {
    if (ng == 16) hipLaunchKernelGGL(srw_finalize_batch_kernel<16>, grid_f, dim3(256), 0, st, fb);
    else hipLaunchKernelGGL(srw_finalize_batch_kernel<4>, grid_f, dim3(256), 0, st, fb);
  }
  return hipGetLastError();
}

}  // namespace srw

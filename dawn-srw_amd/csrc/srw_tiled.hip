// srw_tiled.hip -- bf16 matrix-core SRW forward for wide layers: three tiled
// GEMMs with the gated product P materialised in HBM.
//
// The fused kernels (srw_mfma.hip) keep a [128 tokens x D] fp32 output tile
// in registers for the whole N scan.  At d_model = 1024 (the scaled Know
// pool) that tile is 512 KB, the whole register file of a CU, and the 400M /
// 1B models (D = 1280 / 2048) are larger still.  Here the layer runs as
//
//   pack   W [N, D] -> W^T [D, N64] (unit-contiguous rows, zero tail)
//   stats  S = E.H^T per 256-unit x 256-token tile, rounded to bf16
//          (v41:439) and stored as S [T, N64] bf16; per token and 128 units
//          sum s and sum s^2 (v41:441-442), or (_srw_inference) sum
//          (s - their mean)^2, merged by the tau kernel into the row's
//          centred sum of squares (v41:1719-1721)
//   gate   per tile: XR = R.X^T, the v4.1 gate of the stored scores
//          (v41:506-511) and P = bf16(bf16(g) * bf16(xr)) (v41:516-518),
//          written over S in place; the pass bits and per-token sum gate /
//          sum intensity / active count partials (v41:519-534)
//   write  OUT_c = P[:, chunk c] . W[chunk c, :] per reference chunk c (K =
//          the chunk's units), fp32 partials; the shared finalize rounds each
//          chunk to bf16 and divides by den (v41:518, 584-586)
//
// The reference computes the score GEMM twice (pass 1 and pass 2); here it
// runs once and the bf16 scores travel through HBM: 2 B written + 2 B read
// per (token, unit), plus the same for P, against 2 (dr + 2 D) matrix-core
// flops -- ~770 flop/B at D = 1024, well above the 310 flop/B balance point
// of 2.5 PFLOP/s over 8 TB/s.
//
// All three GEMMs share one main loop: a 256 x 256 output tile per workgroup
// (4 waves as 2 x 2, 128 x 128 = 16 accumulators of 32 x 32 each), operands
// K-contiguous in memory, 64-wide k blocks staged in a double-buffered LDS
// ring by direct global->LDS loads of whole 128-byte lines, 16-byte pieces
// XOR-swizzled by row so the fragment reads are free of bank conflicts.

#include <type_traits>
#include <utility>

#include "srw_internal.hpp"
#include "srw_mfma_util.hpp"

namespace srw {

namespace {

constexpr int kGThreads = 256;              // 4 waves
constexpr int kGRows = 256;                 // rows per operand tile = output tile side
constexpr int kGK = 64;                     // k per stage: one 128-byte line per row
constexpr int kOpBytes = kGRows * kGK * 2;  // 32 KB
constexpr int kStageBytes = 2 * kOpBytes;   // A and B tiles
constexpr int kGemmLds = 2 * kStageBytes;   // two stages: 128 KB
constexpr int kGroupBytes = 32 * kGK * 2;   // 32 rows: one MFMA operand's rows
constexpr int kNAlign = 64;                 // padding of the stored [., N] / [., T] rows

// An operand tile in LDS: 32-row groups of 4 KB; row u of a group at
// (u / 8) * 1 KB + (u % 8) * 128 B, its 16-byte piece q in slot q ^ gswz(u).
__device__ inline int gswz(int u) { return (u & 7) ^ ((u >> 3) & 1); }

// The eight rows a wave loads per stage: rows 32 i + 8 wave + lane / 8 of the
// tile (i = 0..7), 16 bytes each per lane.  Memory row of tile row r =
// min(row0 + r, rows - 1) / div (div = 2 maps paired-route rows to x rows).
struct Opnd {
  const char* base;  // byte address of memory row row0 / div, k = 0 (uniform)
  uint32_t off[8];   // per-lane byte offsets from base: row and swizzled piece
};

__device__ inline Opnd make_opnd(const uint16_t* p, int64_t ld, int64_t row0, int64_t rows, int div, int wave,
                                 int lane) {
  Opnd o;
  const int64_t base_row = row0 / div;
  o.base = reinterpret_cast<const char*>(p + base_row * ld);
  const int r8 = lane >> 3;
  const int piece = (lane & 7) ^ r8 ^ (wave & 1);  // gswz(8 wave + r8) = r8 ^ (wave & 1)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int64_t row = row0 + 32 * i + 8 * wave + r8;
    row = row < rows ? row : rows - 1;
    o.off[i] = static_cast<uint32_t>(((row / div - base_row) * ld + 8 * piece) * 2);
  }
  return o;
}

// acc[i][j] += A-tile rows (128 wa + 32 i ..) . B-tile rows (128 wb + 32 j ..)^T over
// k in [k0, k0 + 64 nk), wave = 2 wa + wb.  hook(kb, stage) runs once block kb
// has landed in LDS, before any wave reads it (all threads call it).
//
// Per 64-wide block: four k-steps of 16 MFMAs.  Operand fragments are double
// buffered in registers: k-step m's MFMAs run while k-step m+1's eight
// fragments are read (one read per two MFMAs, in the order they are used).
// The block barrier sits before k-step 3, whose fragments are then in
// registers: after it no wave reads block kb's stage, so block kb + 2's loads
// go into it at once, one per MFMA of k-step 3 (about four k-steps before
// they are needed), and k-step 3's MFMAs also cover the first fragment reads
// of block kb + 1.  (Global->LDS loads interleaved with fragment reads make
// the compiler wait for every LDS read, so they stay in k-step 3.)
// s_waitcnt immediate for vmcnt(n) (expcnt and lgkmcnt not waited on)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// NBF: B fragments per wave and k-step -- the B tile holds 64 NBF rows (256 or
// 192), each wave 32 NBF of them, so the output tile is 256 x 64 NBF (192 when
// the B side is 384 wide: no padded columns).
template <int NBF, class Hook>
__device__ inline void gemm_loop(f32x16_t (&acc)[4][NBF], const Opnd& A, const Opnd& B, int64_t k0, int nk,
                                 char* lds, int wave, int lane, Hook&& hook) {
  constexpr int NB = 64 * NBF;                 // B-tile rows
  constexpr int NL = 8 + NB / 32;              // 16-byte loads per wave and k block
  constexpr int NQ = 4 * NBF;                  // MFMAs per wave and k-step
  constexpr int NF = 4 + NBF;                  // operand fragments per k-step
  constexpr int STAGE = kOpBytes + NB * kGK * 2;
  const int wa = wave >> 1, wb = wave & 1;
  const int u = lane & 31, h = lane >> 5;
  int le[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) le[m] = (u >> 3) * 1024 + (u & 7) * 128 + (((2 * m + h) ^ gswz(u)) * 16);
  // block b's loads (blocks past the last reload the last one: in bounds, never used)
  auto issue = [&](int q, int b, char* stage) {
    const int64_t kbyte = (k0 + static_cast<int64_t>(b < nk ? b : nk - 1) * kGK) * 2;
    if (q < 8)
      g2lds16(A.base + kbyte + A.off[q], stage + q * kGroupBytes + wave * 1024);
    else
      g2lds16(B.base + kbyte + B.off[q - 8], stage + kOpBytes + (q - 8) * kGroupBytes + wave * 1024);
  };
  // fragment g of k-step m: g < 4 the A rows 128 wa + 32 g .., else the B rows 32 NBF wb + 32 (g - 4) ..
  auto frag = [&](const char* stage, int g, int m) {
    const int off = g < 4 ? (4 * wa + g) * kGroupBytes : kOpBytes + (NBF * wb + g - 4) * kGroupBytes;
    return *reinterpret_cast<const u32x4_t*>(stage + off + le[m]);
  };
  // the order the next k-step uses its fragments: a0, b0 .. b(NBF-1), a1, a2, a3
  auto order = [](int r) { return r == 0 ? 0 : (r <= NBF ? 3 + r : r - NBF); };
#pragma unroll
  for (int q = 0; q < NL; ++q) issue(q, 0, lds);
#pragma unroll
  for (int q = 0; q < NL; ++q) issue(q, 1, lds + STAGE);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(NL));  // block 0 has landed, block 1 is in flight
  barrier_lds();
  hook(0, lds);
  u32x4_t f[2][NF];
#pragma unroll
  for (int g = 0; g < NF; ++g) f[0][g] = frag(lds, g, 0);
  for (int kb = 0; kb < nk; ++kb) {
    char* st = lds + (kb & 1) * STAGE;
    char* nxt = lds + ((kb & 1) ^ 1) * STAGE;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int cb = m & 1;
      if (m == 3) {
        __builtin_amdgcn_sched_barrier(0);
        wait_vm0();
        __syncthreads();  // block kb + 1 has landed; nobody reads block kb's stage any more
        if (kb + 1 < nk) hook(kb + 1, nxt);
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        acc[q / NBF][q % NBF] = mfma(f[cb][q / NBF], f[cb][4 + q % NBF], acc[q / NBF][q % NBF]);
        // fragment r of the next k-step is read at MFMA r NQ / NF (one per two MFMAs at NBF = 4)
#pragma unroll
        for (int r = 0; r < NF; ++r) {
          if (r * NQ / NF == q) {
            const int g = order(r);
            f[cb ^ 1][g] = m < 3 ? frag(st, g, m + 1) : frag(nxt, g, 0);
          }
        }
        if (m == 3) {
#pragma unroll
          for (int L = q * NL / NQ; L < (q + 1) * NL / NQ; ++L) issue(L, kb + 2, st);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  wait_vm0();
  __syncthreads();  // the trailing reloads have landed before LDS is reused
}

// LDS of a gemm_loop<NBF> workgroup: two stages of the A and B tiles
constexpr int gemm_lds(int nbf) { return 2 * (kOpBytes + 64 * nbf * kGK * 2); }

struct NoHook {
  __device__ void operator()(int, char*) const {}
};

// Workgroup -> (row tile, column tile) with the column tile shared by the
// workgroups of one XCD (blockIdx % 8 on MI355X): they walk the row tiles of
// one column tile together, so its operand rows are fetched into that XCD's
// L2 once.  Returns false for the padding workgroups of the last group.
__device__ inline bool tile_of(int nrow, int ncol, int& rt, int& ct) {
  const int x = blockIdx.x & 7, k = blockIdx.x >> 3;
  ct = (k / nrow) * 8 + x;
  rt = k % nrow;
  return ct < ncol;
}

// ---------------------------------------------------------------------------
// pack: W [N, D] -> W^T [D, N64], zero for units >= N
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_wt_kernel(const uint16_t* __restrict__ W, uint16_t* __restrict__ WT,
                                                      int64_t N, int64_t N64, int D) {
  __shared__ uint16_t tile[64][66];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int d0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t n = n0 + r;
    const int d = d0 + tx;
    tile[r][tx] = (n < N && d < D) ? W[n * D + d] : static_cast<uint16_t>(0);
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int d = d0 + r;
    const int64_t n = n0 + tx;
    if (d < D && n < N64) WT[static_cast<int64_t>(d) * N64 + n] = tile[tx][r];
  }
}

// ---------------------------------------------------------------------------
// stats: per-token moment partials of the bf16 scores
// ---------------------------------------------------------------------------
struct TStatsParams {
  const uint16_t* h;    // [Tv, dr]
  const uint16_t* emb;  // [N, dr]
  uint16_t* S;          // [Tv, N64] bf16 scores (zero for units >= N)
  float* mom;           // [2 CT][Tv][2]: per 128 units (sum s, sum s^2), or (sum s, sum (s - their mean)^2)
  int64_t Tv, N, N64, dr;
  int RT, CT;
  int centred;          // second moments about the 128 units' own mean (merged by srw_tau_kernel's kTauChan)
};

__global__ __launch_bounds__(kGThreads) void tiled_stats_kernel(TStatsParams p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wa = wave >> 1, wb = wave & 1, u = lane & 31, h = lane >> 5;
  int rt, ct;
  if (!tile_of(p.RT, p.CT, rt, ct)) return;
  const int64_t u0 = static_cast<int64_t>(ct) * kGRows, v0 = static_cast<int64_t>(rt) * kGRows;
  const Opnd A = make_opnd(p.emb, p.dr, u0, p.N, 1, wave, lane);
  const Opnd B = make_opnd(p.h, p.dr, v0, p.Tv, 1, wave, lane);
  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};
  gemm_loop(acc, A, B, 0, static_cast<int>(p.dr / kGK), lds, wave, lane, NoHook{});

  const int64_t nleft = p.N - (u0 + 128 * wa + 4 * h);  // units of this wave-row left in the pool
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t t = v0 + 128 * wb + 32 * j + u;
    uint16_t* srow = p.S + t * p.N64;
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int v = 0; v < 16; v += 4) {
        uint32_t sq[2];
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          const uint32_t sp = pack_bf16(acc[i][j][v + 2 * e2], acc[i][j][v + 2 * e2 + 1]);  // bf16 scores (v41:439)
          float a = lo_f32(sp), b = hi_f32(sp);
          const int r = 32 * i + 8 * (v >> 2) + 2 * e2;  // unit offset from u0 + 128 wa + 4 h
          const bool oka = r < nleft, okb = r + 1 < nleft;
          a = oka ? a : 0.f;
          b = okb ? b : 0.f;
          s1 += a;
          s2 += __fmul_rn(a, a);
          s1 += b;
          s2 += __fmul_rn(b, b);
          sq[e2] = pack_bf16(a, b);
        }
        const int64_t n0 = u0 + 128 * wa + 32 * i + 8 * (v >> 2) + 4 * h;
        if (t < p.Tv && n0 < p.N64) {
          typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2_t*>(srow + n0) = u32x2_t{sq[0], sq[1]};
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    s1 += __shfl_xor(s1, 32);
    if (p.centred) {
      // sum (s - mean)^2 over these units' bf16 scores, their mean from s1
      // (v41:1719-1721 over a 128-unit slice; merged in srw_tau_kernel)
      const int64_t nrow = p.N - (u0 + 128 * wa);
      const float n = static_cast<float>(nrow <= 0 ? 0 : (nrow < 128 ? nrow : 128));
      const float mu = n > 0.f ? s1 / n : 0.f;
      s2 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const uint32_t sp = pack_bf16(acc[i][j][v], acc[i][j][v + 1]);
          const int r = 32 * i + 8 * (v >> 2) + (v & 3);
          const float da = r < nleft ? lo_f32(sp) - mu : 0.f, db = r + 1 < nleft ? hi_f32(sp) - mu : 0.f;
          s2 += __fmul_rn(da, da);
          s2 += __fmul_rn(db, db);
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
struct TGateParams {
  const uint16_t* x;     // [T, D] (row v / routes)
  const uint16_t* read;  // [N, D]
  const float* tau;      // [Tv]
  uint16_t* P;           // [Tv, N64]: the bf16 scores in, P out (in place)
  uint16_t* P_out;       // KEEP: P here instead, the scores stay in P
  uint16_t* XR_out;      // KEEP: bf16 x.r [Tv, N64]
  float* tok_part;       // [2 CT][Tv][4]: sum gate, sum intensity, active count
  uint32_t* mask32;      // [Tv][mask_words32] or null
  float* G;              // [Tv, N] every unit's fp32 gate (SRW_FLAG_GATE_OUT) or null
  int64_t mask_words32;
  int64_t Tv, N, N64, D;
  int routes, RT, CT;
  GateParams gp;
  float exp_scale;       // -sharpness * log2(e)
};

// The v4.1 gate of one bf16 score in the folded form (v41:503-511):
// arg = s c + k (c = -sharpness log2 e, k = -(tau + thr) c), act = 1 / (1 +
// 2^arg), intensity = eps + min(max(s - tau - thr - cut, 0), maxi), g = act
// intensity; the sign bit of arg is the pass bit.  The product stays a
// rounded multiply (no contraction into a caller's running sum), so the
// dense gate kernel and the sparse mark kernel sum the same gate values.
struct GateElem {
  float g, inten;
  uint32_t sign;
};
__device__ inline GateElem gate_elem(float s, float c_exp, float k_exp, float tau_cut, float eps, float maxi) {
#pragma clang fp contract(off)
  const float arg = fmaf(s, c_exp, k_exp);
  const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(arg));
  const float inten = eps + __builtin_amdgcn_fmed3f(s - tau_cut, 0.0f, maxi);
  return GateElem{act * inten, inten, __float_as_uint(arg)};
}

// KEEP (the backward's recompute): P and x.r go to P_out / XR_out and the
// stored scores stay.  GOUT: every unit's fp32 gate also goes to G (a
// variant of its own: the per-element stores and their addresses would
// otherwise sit in every call's epilogue code).
template <bool KEEP, bool GOUT = false>
__global__ __launch_bounds__(kGThreads) void tiled_gate_kernel(TGateParams p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wa = wave >> 1, wb = wave & 1, u = lane & 31, h = lane >> 5;
  int rt, ct;
  if (!tile_of(p.RT, p.CT, rt, ct)) return;
  const int64_t u0 = static_cast<int64_t>(ct) * kGRows, v0 = static_cast<int64_t>(rt) * kGRows;
  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};
  {
    const Opnd A = make_opnd(p.read, p.D, u0, p.N, 1, wave, lane);
    const Opnd B = make_opnd(p.x, p.D, v0, p.Tv, p.routes, wave, lane);
    gemm_loop(acc, A, B, 0, static_cast<int>(p.D / kGK), lds, wave, lane, NoHook{});
  }

  // gate epilogue (v41:503-534): margin = s - tau - thr folded into
  // arg = s * c + k (c = -sharpness log2 e), sigmoid = 1 / (1 + 2^arg),
  // intensity = eps + min(max(s - tau - thr - cut, 0), maxi);
  // P = bf16(bf16(g) * bf16(xr)), four consecutive units per load / store.
  // FULL: every unit of the tile is in the pool (all but the last unit tile).
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  const int64_t nleft = p.N - (u0 + 128 * wa + 4 * h);  // units of this wave-row left in the pool
  const float c_exp = p.exp_scale, eps = p.gp.eps, maxi = p.gp.maxi;
  auto epilogue = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = v0 + 128 * wb + 32 * j + u;
      const bool tok = t < p.Tv;
      uint16_t* prow = p.P + (tok ? t : p.Tv - 1) * p.N64;
      const float tau_thr = p.tau[tok ? t : p.Tv - 1] + p.gp.thr;
      const float k_exp = -tau_thr * c_exp;
      const float tau_cut = tau_thr + p.gp.cut;
      float gs = 0.f, is = 0.f;
      int na = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t nb = u0 + 128 * wa + 32 * i + 4 * h;
        u32x2_t sv[4], xv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)  // the last unit tile may reach past the row's N64 columns
          sv[q] = FULL || nb + 8 * q < p.N64 ? *reinterpret_cast<const u32x2_t*>(prow + nb + 8 * q) : u32x2_t{0u, 0u};
        uint32_t bits = 0;  // element v of the 16 at bit 15 - v: set <=> arg < 0 <=> act > 0.5
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const uint32_t sp = sv[v >> 2][(v >> 1) & 1];  // bf16 scores of units v, v + 1
          float g2[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const GateElem ge = gate_elem(e ? hi_f32(sp) : lo_f32(sp), c_exp, k_exp, tau_cut, eps, maxi);
            float g = ge.g, inten = ge.inten;
            uint32_t sign = ge.sign;
            if constexpr (!FULL) {  // units past N count for nothing
              const bool ok = 32 * i + 8 * ((v + e) >> 2) + ((v + e) & 3) < nleft;
              g = ok ? g : 0.f;
              inten = ok ? inten : 0.f;
              sign = ok ? sign : 0u;
            }
            gs += g;
            is += inten;
            bits = __builtin_amdgcn_alignbit(bits, sign, 31);  // bits << 1 | sign bit
            g2[e] = g;
            if constexpr (GOUT) {
              const int64_t un = nb + 8 * ((v + e) >> 2) + ((v + e) & 3);
              if (tok && un < p.N) p.G[t * p.N + un] = g;
            }
          }
          const uint32_t gq = pack_bf16(g2[0], g2[1]);                              // gate_bf (v41:516)
          const uint32_t xq = pack_bf16(acc[i][j][v], acc[i][j][v + 1]);            // xr (v41:517)
          if constexpr (KEEP) xv[v >> 2][(v >> 1) & 1] = xq;
          sv[v >> 2][(v >> 1) & 1] = pack_bf16(lo_f32(gq) * lo_f32(xq), hi_f32(gq) * hi_f32(xq));  // (v41:518)
        }
        if (tok) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (!(FULL || nb + 8 * q < p.N64)) continue;
            if constexpr (KEEP) {
              *reinterpret_cast<u32x2_t*>(p.P_out + t * p.N64 + nb + 8 * q) = sv[q];
              *reinterpret_cast<u32x2_t*>(p.XR_out + t * p.N64 + nb + 8 * q) = xv[q];
            } else {
              *reinterpret_cast<u32x2_t*>(prow + nb + 8 * q) = sv[q];
            }
          }
        }
        // element v -> unit 8 (v / 4) + 4 h + v % 4 of the 32-unit block
        const uint32_t b = __builtin_bitreverse32(bits) >> 16;  // element v at bit v
        uint32_t m = (b & 0xFu) | ((b & 0xF0u) << 4) | ((b & 0xF00u) << 8) | ((b & 0xF000u) << 12);
        m <<= 4 * h;
        na += __builtin_popcount(m);
        m |= __shfl_xor(m, 32);
        const int64_t word = (u0 + 128 * wa + 32 * i) / 32;
        if (p.mask32 && h == 0 && tok && word < p.mask_words32) p.mask32[t * p.mask_words32 + word] = m;
        __builtin_amdgcn_sched_barrier(0);  // one accumulator at a time: keeps the live registers bounded
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
  };
  if (u0 + kGRows <= p.N)
    epilogue(std::integral_constant<bool, true>{});
  else
    epilogue(std::integral_constant<bool, false>{});
}

// ---------------------------------------------------------------------------
// Sparse skip (SRW_FLAG_SPARSE_SKIP) at prefill sizes.  The score GEMM runs
// dense (the stats kernel, S stored); then
//   mark    the gate of every (token, unit) from the stored scores -- the
//           gate kernel's epilogue without its GEMM: the same pass bits and
//           per-token partial sums, so gate_sum, den, n_active and the mask
//           equal the dense path's bit for bit -- plus, per 32-token tile,
//           the union of the units some token passes (v41:505-511: margin >
//           0 <=> act > 0.5)
//           and the bf16 gates of the union's units, 32 tokens contiguous
//           per unit (G: the union units of each 128-unit slice packed at
//           the slice's start)
//   list    per 32-token tile, the union compacted into an index list (and
//           each entry's slot in G), with the reference chunks' boundaries
//   gather  per 32-token tile, the read and write GEMMs over the union's
//           units only, 32 at a time: their R and W rows gathered, x.R^T
//           split over eight waves' k-slabs and summed in LDS, P =
//           bf16(bf16(g) bf16(xr)) with the gates from G, OUT += P . W; one
//           fp32 partial per reference chunk for the shared finalize.
// Units no token of a tile passes are left out of out only (their gates are
// epsilon-sized: act < 0.5 and intensity = eps, v41:509-511); the sums, den
// and the mask keep them.
// ---------------------------------------------------------------------------
struct SpMarkParams {
  const uint16_t* S;     // [Tv, N64] bf16 scores
  const float* tau;      // [Tv]
  float* tok_part;       // [2 CT][Tv][4] as the gate kernel's
  uint32_t* mask32;      // [Tv][mask_words32] or null
  uint32_t* uni;         // [TT32][W32]: units some token of the 32-token tile passes
  uint16_t* G;           // [TT32][GS][32]: bf16 gates, slice sl's union units at slots 128 sl + rank
  int64_t mask_words32, W32, GS;
  int64_t Tv, N, N64;
  int CT;
  GateParams gp;
  float exp_scale;
};

// One wave per (32 tokens, 128-unit slice): lane u + 32 h holds token 32
// tile + u and the slice's units 32 i + 8 (v / 4) + 4 h + v % 4 -- the gate
// kernel's epilogue layout and arithmetic.
__global__ __launch_bounds__(256) void sp_mark_kernel(SpMarkParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int u = lane & 31, h = lane >> 5;
  const int nsl = 2 * p.CT;                      // 128-unit slices (the gate kernel's partials)
  const int sgroups = (nsl + 3) / 4;
  const int tile = blockIdx.x / sgroups;
  const int sl = (blockIdx.x % sgroups) * 4 + wave;
  if (sl >= nsl) return;
  const int64_t t = static_cast<int64_t>(tile) * 32 + u;
  const bool tok = t < p.Tv;
  const uint16_t* prow = p.S + (tok ? t : p.Tv - 1) * p.N64;
  const float c_exp = p.exp_scale, eps = p.gp.eps, maxi = p.gp.maxi;
  const float tau_thr = p.tau[tok ? t : p.Tv - 1] + p.gp.thr;
  const float k_exp = -tau_thr * c_exp;
  const float tau_cut = tau_thr + p.gp.cut;
  const int64_t u0 = static_cast<int64_t>(sl) * 128;
  const int64_t nleft = p.N - (u0 + 4 * h);
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  uint16_t* gtile = p.G + (static_cast<int64_t>(tile) * p.GS + static_cast<int64_t>(sl) * 128) * 32 + u;
  float gs = 0.f, is = 0.f;
  int na = 0, gbase = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t nb = u0 + 32 * i + 4 * h;
    u32x2_t sv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) sv[q] = nb + 8 * q < p.N64 ? *reinterpret_cast<const u32x2_t*>(prow + nb + 8 * q) : u32x2_t{0u, 0u};
    uint32_t bits = 0;
    uint32_t gq[8];  // bf16 gates of elements 2 k, 2 k + 1
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      const uint32_t sp = sv[v >> 2][(v >> 1) & 1];
      float g2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const GateElem ge = gate_elem(e ? hi_f32(sp) : lo_f32(sp), c_exp, k_exp, tau_cut, eps, maxi);
        float g = ge.g, inten = ge.inten;
        uint32_t sign = ge.sign;
        const bool ok = 32 * i + 8 * ((v + e) >> 2) + ((v + e) & 3) < nleft;  // units past N count for nothing
        g = ok ? g : 0.f;
        inten = ok ? inten : 0.f;
        sign = ok ? sign : 0u;
        gs += g;
        is += inten;
        bits = __builtin_amdgcn_alignbit(bits, sign, 31);
        g2[e] = g;
      }
      gq[v >> 1] = pack_bf16(g2[0], g2[1]);  // gate_bf (v41:516)
    }
    const uint32_t b = __builtin_bitreverse32(bits) >> 16;  // element v at bit v
    uint32_t m = (b & 0xFu) | ((b & 0xF0u) << 4) | ((b & 0xF00u) << 8) | ((b & 0xF000u) << 12);
    m <<= 4 * h;
    na += __builtin_popcount(m);
    m |= __shfl_xor(m, 32);
    const int64_t word = (u0 + 32 * i) / 32;
    if (p.mask32 && h == 0 && tok && word < p.mask_words32) p.mask32[t * p.mask_words32 + word] = m;
    // the union over the tile's tokens
    uint32_t um = tok ? m : 0u;
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) um |= __shfl_xor(um, o);
    if (lane == 0 && word < p.W32) p.uni[static_cast<int64_t>(tile) * p.W32 + word] = um;
    // the union units' gates: unit w of the word at slot gbase + (union units below w)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int w = 8 * (v >> 2) + 4 * h + (v & 3);
      if ((um >> w) & 1u) {
        const int slot = gbase + __builtin_popcount(um & ((1u << w) - 1u));
        gtile[slot * 32] = static_cast<uint16_t>((v & 1) ? gq[v >> 1] >> 16 : gq[v >> 1] & 0xffffu);
      }
    }
    gbase += __builtin_popcount(um);
  }
  gs += __shfl_xor(gs, 32);
  is += __shfl_xor(is, 32);
  na += __shfl_xor(na, 32);
  if (h == 0 && tok) {
    float* tp = p.tok_part + (static_cast<int64_t>(sl) * p.Tv + t) * 4;
    tp[0] = gs;
    tp[1] = is;
    tp[2] = static_cast<float>(na);
    tp[3] = 0.f;
  }
}

// Per 32-token tile: its union's units in increasing order, list[tile][k],
// and cstart[tile][c] = the list position of the first unit of reference
// chunk c (c = 0..nc; cstart[nc] = the count).  One workgroup per tile, 256
// union words per round, an exclusive scan of their popcounts.
__global__ __launch_bounds__(256) void sp_list_kernel(const uint32_t* __restrict__ uni, int64_t W32, int64_t N,
                                                      int64_t cs, int nc, int32_t* __restrict__ list,
                                                      int32_t* __restrict__ glist, int32_t* __restrict__ cstart) {
  __shared__ int wsum[4];
  const int tile = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t* uw = uni + static_cast<int64_t>(tile) * W32;
  int32_t* out = list + static_cast<int64_t>(tile) * N;
  int32_t* gout = glist + static_cast<int64_t>(tile) * N;
  int32_t* cst = cstart + static_cast<int64_t>(tile) * (nc + 1);
  int base = 0;
  for (int64_t w0 = 0; w0 < W32; w0 += 256) {
    const int64_t w = w0 + tid;
    const uint32_t bits = w < W32 ? uw[w] : 0u;
    const int pc = __builtin_popcount(bits);
    // inclusive scan over the wave, then over the waves
    int x = pc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int before = base;
    for (int k = 0; k < wave; ++k) before += wsum[k];
    const int start = before + x - pc;  // this word's first list position
    // the slot in G: 128 (w / 4) + the entry's rank among its 128-unit slice's
    // union units (the slice's first word is handled by lane & ~3)
    const int sfirst = __shfl(start, lane & ~3);
    const int gslot = static_cast<int>(w / 4) * 128 + (start - sfirst);
    uint32_t b = bits;
    int k = 0;
    while (b) {
      const int bit = __builtin_ctz(b);
      out[start + k] = static_cast<int32_t>(w * 32 + bit);
      gout[start + k] = gslot + k;
      b &= b - 1;
      ++k;
    }
    // chunk boundaries inside this word's 32 units
    for (int c = 1; c < nc; ++c) {
      const int64_t bu = c * cs;
      if (bu / 32 == w) cst[c] = start + __builtin_popcount(bits & ((1u << (bu % 32)) - 1u));
    }
    const int total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();  // wsum is rewritten next round
    base += total;
  }
  if (tid == 0) {
    cst[0] = 0;
    cst[nc] = base;
  }
}

// The gathered read and write GEMMs of one 32-token tile over the listed
// units of one reference chunk (one workgroup, eight waves; workgroups in
// chunk-major order), in blocks of 32 listed units.  Wave w owns the read
// GEMM's k-slab [w D / 8, (w + 1) D / 8) (its x fragments in LDS) and the
// output columns of the same range: lane l holds columns w D / 8 + F (l % 32)
// + f, f < F, so that one 2F-byte load of a W row gives a lane its F columns
// of one unit.  Per block:
//   XR^T = R_blk . X^T over the slab (A: the units' R rows, 16-byte loads),
//   the eight partial accumulators summed in LDS in wave order; each wave
//   takes 1 / 8 of the 32 x 32 elements (accumulator registers 2 w, 2 w + 1),
//   their bf16 gates from G, and writes P = bf16(bf16(g) bf16(xr)) in the
//   write GEMM's A-operand order (unit_of_k == unit_of_acc) back to LDS;
//   OUT += P . W_blk, the B fragments (8 units x 1 column) assembled in
//   registers from the eight units' 2F-byte row pieces.
// Software pipeline: the next block's W pieces, gates and R rows are
// requested during the current block, the list entries two blocks ahead;
// lane l keeps unit l % 32 of a block and the other lanes' units come by
// cross-lane shuffles.  OUT goes to out_part[chunk] (zeros for a
// chunk none of whose units is listed).
template <int F>  // D = 256 F
struct SpGemm {
  static constexpr int D = 256 * F;
  static constexpr int KS = 2 * F;  // the read GEMM's k-steps per wave (D / 8 / 16)
};
struct SpGatherParams {
  const uint16_t* x;     // [T, D] (row v / routes)
  const uint16_t* read;  // [N, D]
  const uint16_t* write; // [N, D]
  const uint16_t* G;     // [TT32][GS][32] the union units' bf16 gates (sp_mark_kernel)
  const int32_t* list;   // [TT32][N] units
  const int32_t* glist;  // [TT32][N] their slots in G
  const int32_t* cstart; // [TT32][nc + 1]
  float* out_part;       // [nc][Tv][D]
  int64_t Tv, N, GS;
  int routes, nc, TT32;
};
constexpr int kSpThreads = 512;

// lane's list entry at position k of [.., bend) (-1: padding past the end) and its slot in G
struct SpEntry {
  int32_t u, g;
};
__device__ inline SpEntry sp_entry(const int32_t* lst, const int32_t* glst, int k, int bend) {
  if (k < bend) return SpEntry{lst[k], glst[k]};
  return SpEntry{-1, 0};
}

template <int F>
struct SpPiece;  // F bf16 of one W row
template <>
struct SpPiece<1> {
  typedef uint16_t T;
  __device__ static uint32_t at(T v, int) { return v; }
};
template <>
struct SpPiece<2> {
  typedef uint32_t T;
  __device__ static uint32_t at(T v, int f) { return f ? v >> 16 : v & 0xffffu; }
};
template <>
struct SpPiece<4> {
  typedef uint32_t T __attribute__((ext_vector_type(2)));
  __device__ static uint32_t at(T v, int f) { return (f & 1) ? v[f >> 1] >> 16 : v[f >> 1] & 0xffffu; }
};

template <int F>
__global__ __launch_bounds__(kSpThreads, 1) void sp_gather_kernel(SpGatherParams p) {
  constexpr int D = SpGemm<F>::D, KS = SpGemm<F>::KS;
  typedef typename SpPiece<F>::T piece_t;
  __shared__ u32x4_t xs[8][KS][64];  // wave w's x fragments (B operand of XR^T), [k-step][lane]
  __shared__ float4 part[8][4][64];  // wave q's x.r partial: [q][v / 4][lane] = elements 4 (v / 4) .. + 3
  __shared__ uint32_t pl[8][64];     // P: [w][lane] = elements 2 w, 2 w + 1 (A operand of the write GEMM)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, half = lane >> 5;
  // chunk-major: the workgroups resident at one time work on the same
  // reference chunk, so that each XCD's L2 serves the R / W rows they share
  const int c = blockIdx.x / p.TT32, tile = blockIdx.x % p.TT32;
  const int64_t t = static_cast<int64_t>(tile) * 32 + col;
  const int64_t tl = t < p.Tv ? t : p.Tv - 1;
  const int32_t* lst = p.list + static_cast<int64_t>(tile) * p.N;
  const int32_t* glst = p.glist + static_cast<int64_t>(tile) * p.N;
  const int32_t* cs = p.cstart + static_cast<int64_t>(tile) * (p.nc + 1);
  const int b_lo = cs[c], b_hi = cs[c + 1];
  const int k0 = wave * (D / 8);  // this wave's k-slab and output columns
  // x of this wave's k-slab (B operand of XR^T: lane l, token l % 32), kept
  // in LDS (each wave reads back only its own fragments)
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    xs[wave][ks][lane] = *reinterpret_cast<const u32x4_t*>(p.x + (tl / p.routes) * D + k0 + 16 * ks + 8 * half);
  const uint16_t* gcol = p.G + static_cast<int64_t>(tile) * p.GS * 32 + col;  // this lane's token in G
  // R / W rows by 32-bit byte offsets from the wave's (uniform) slab base
  const char* rbase = reinterpret_cast<const char*>(p.read + k0);
  const char* wbase = reinterpret_cast<const char*>(p.write + k0);
  const uint32_t rlane = 16u * half, wlane = 2u * F * col;
  const uint32_t gsh = 16u * (col & 1);  // this lane's gate in a token pair's 4 bytes
  f32x16_t oacc[F];
#pragma unroll
  for (int f = 0; f < F; ++f) oacc[f] = f32x16_t{};
  // a block's W row pieces (unit unit_of_k(j, half, i) of the block), the
  // bf16 gates of this lane's elements 2 wave, 2 wave + 1 (padding: 0)
  struct BlockLoads {
    piece_t wp[2][8];
    uint32_t q0, q1;  // 4-byte loads of the gates of this lane's token pair (taken apart where used)
    bool pad0, pad1;
  };
  auto issue = [&](const SpEntry& e, BlockLoads& bl) {
    // all shuffles first, then all loads: one wait for the shuffles
    int32_t wu[2][8], gs[2], un[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) wu[j][i] = __shfl(e.u, unit_of_k(j, half, i));
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      gs[q] = __shfl(e.g, unit_of_acc(2 * wave + q, half));
      un[q] = __shfl(e.u, unit_of_acc(2 * wave + q, half));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        bl.wp[j][i] = *reinterpret_cast<const piece_t*>(
            wbase + (static_cast<uint32_t>(wu[j][i] >= 0 ? wu[j][i] : 0) * (2u * D) + wlane));
    // (4-byte loads, no 16-bit extension next to the load; padding entries: slot 0)
    const uint32_t* gp = reinterpret_cast<const uint32_t*>(gcol - (col & 1));
    bl.q0 = gp[static_cast<int64_t>(gs[0]) * 16];
    bl.q1 = gp[static_cast<int64_t>(gs[1]) * 16];
    bl.pad0 = un[0] < 0;
    bl.pad1 = un[1] < 0;
  };

  // ping-pong (no register copies, which would wait for loads in flight):
  // the current block's loads and the next one's; the next block's list
  // entries and the ones after
  SpEntry ul_a = sp_entry(lst, glst, b_lo + 32 + col, b_hi), ul_b;
  u32x4_t rf[KS];
  BlockLoads bl_a, bl_b;
  {
    const SpEntry e = sp_entry(lst, glst, b_lo + col, b_hi);
    const uint32_t ro = static_cast<uint32_t>(e.u >= 0 ? e.u : 0) * (2u * D) + rlane;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) rf[ks] = *reinterpret_cast<const u32x4_t*>(rbase + ro + 32 * ks);
    issue(e, bl_a);
  }
  // one block: the next block's W pieces, gates and R rows are requested
  // into `nxt` / rf while this block (`cur`, rf) is computed
  auto block = [&](int b0, const BlockLoads& cur, BlockLoads& nxt, const SpEntry& ul_nxt, SpEntry& ul_nx2) {
    __builtin_amdgcn_sched_barrier(0);  // nothing of the next block moves up into this one
    issue(ul_nxt, nxt);
    ul_nx2 = sp_entry(lst, glst, b0 + 64 + col, b_hi);  // list entries two blocks ahead
    // read GEMM over this wave's k-slab
    f32x16_t racc = {};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) racc = mfma(rf[ks], xs[wave][ks][lane], racc);
    // the next block's R rows
    {
      const uint32_t ro = static_cast<uint32_t>(ul_nxt.u >= 0 ? ul_nxt.u : 0) * (2u * D) + rlane;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) rf[ks] = *reinterpret_cast<const u32x4_t*>(rbase + ro + 32 * ks);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) part[wave][g][lane] = float4{racc[4 * g], racc[4 * g + 1], racc[4 * g + 2], racc[4 * g + 3]};
    __syncthreads();
    // elements 2 wave, 2 wave + 1: x.r summed over the k-slabs in order, the
    // bf16 gates from G (v41:503-518)
    {
      float xr2[2];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float2 v2 = reinterpret_cast<const float2*>(&part[q][wave >> 1][lane])[wave & 1];
        xr2[0] = q ? xr2[0] + v2.x : v2.x;
        xr2[1] = q ? xr2[1] + v2.y : v2.y;
      }
      const uint32_t xq2 = pack_bf16(xr2[0], xr2[1]);                                   // bf16 x.r (v41:517)
      const uint32_t g2 = ((cur.q0 >> gsh) & 0xffffu) | ((cur.q1 >> gsh) << 16);
      const uint32_t gq = g2 & ((cur.pad0 ? 0u : 0xffffu) | (cur.pad1 ? 0u : 0xffff0000u));  // gate_bf (v41:516)
      pl[wave][lane] = pack_bf16(lo_f32(gq) * lo_f32(xq2), hi_f32(gq) * hi_f32(xq2));  // (v41:518)
    }
    __syncthreads();
    // write GEMM: OUT[32 tokens x this wave's columns] += P . W_blk
    const u32x4_t a0 = {pl[0][lane], pl[1][lane], pl[2][lane], pl[3][lane]};
    const u32x4_t a1 = {pl[4][lane], pl[5][lane], pl[6][lane], pl[7][lane]};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int f = 0; f < F; ++f) {
        u32x4_t bf;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          bf[e] = SpPiece<F>::at(cur.wp[j][2 * e], f) | (SpPiece<F>::at(cur.wp[j][2 * e + 1], f) << 16);
        oacc[f] = mfma(j ? a1 : a0, bf, oacc[f]);
      }
    }
  };
  // blocks in pairs; past the end a block is all padding (zero gates: P = 0
  // adds nothing), which keeps the loop body free of a branch whose merge
  // would need register copies
  for (int b0 = b_lo; b0 < b_hi; b0 += 64) {
    block(b0, bl_a, bl_b, ul_a, ul_b);
    block(b0 + 32, bl_b, bl_a, ul_b, ul_a);
  }
  // the chunk's partial (zeros where none of its units is listed); the
  // lane's first token row, register v is row 8 (v / 4) + v % 4 after it
  const bool full_tile = static_cast<int64_t>(tile) * 32 + 32 <= p.Tv;
  const int64_t t0 = static_cast<int64_t>(tile) * 32 + 4 * half;
  float* op = p.out_part + (static_cast<int64_t>(c) * p.Tv + t0) * D + k0 + F * col;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int r = 8 * (v >> 2) + (v & 3);
    if (!full_tile && t0 + r >= p.Tv) continue;
    float* dst = op + r * D;
    if constexpr (F == 4) {
      *reinterpret_cast<float4*>(dst) = float4{oacc[0][v], oacc[1][v], oacc[2][v], oacc[3][v]};
    } else if constexpr (F == 2) {
      *reinterpret_cast<float2*>(dst) = float2{oacc[0][v], oacc[1][v]};
    } else {
      dst[0] = oacc[0][v];
    }
  }
}

// ---------------------------------------------------------------------------
// write: OUT partial of one N-split = P[:, split units] . W^T[:, split units]^T
// ---------------------------------------------------------------------------
struct TWriteParams {
  const uint16_t* P;   // [Tv, N64]
  const uint16_t* wt;  // [D, N64]
  float* out_part;     // [S][Tv][D]
  int64_t Tv, N, N64, D, cs;
  int nc, spc, S, RT, DT;
  int round_out;       // store bf16-rounded values (one split: out_part is the result)
};

// zero the units outside [lo, hi) of the P tile of one k block (first unit kbase)
__device__ inline void mask_units(char* tile, int64_t kbase, int64_t lo, int64_t hi) {
  const int r = threadIdx.x, u = r & 31;
  char* row = tile + (r >> 5) * kGroupBytes + (u >> 3) * 1024 + (u & 7) * 128;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    uint16_t* e = reinterpret_cast<uint16_t*>(row + ((q ^ gswz(u)) * 16));
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t n = kbase + 8 * q + k;
      if (n < lo || n >= hi) e[k] = 0;
    }
  }
}

// MAYROUND: p.round_out is honoured (the backward's products); without it
// the kernel has no rounding code (the forward's write GEMM: its register
// allocation spilled with the rounded form compiled in beside the plain one).
template <int NBF, bool MAYROUND>
__device__ __attribute__((always_inline)) inline void write_body(const TWriteParams& p, const int bid) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wa = wave >> 1, wb = wave & 1, u = lane & 31, h = lane >> 5;
  // workgroups of one (token tile, split) on one XCD, consecutive: their D
  // tiles share the P tile
  const int x = bid & 7, k = bid >> 3;
  const int dt = k % p.DT;
  const int w = (k / p.DT) * 8 + x;
  if (w >= p.RT * p.S) return;
  const int rt = w % p.RT, split = w / p.RT;
  // the split's k blocks: reference chunk c's blocks, divided evenly into spc
  const int c = split / p.spc, sub = split % p.spc;
  const int64_t lo = c * p.cs, hi = (c + 1) * p.cs < p.N ? (c + 1) * p.cs : p.N;
  const int64_t b_lo = lo / kGK, b_hi = (hi + kGK - 1) / kGK, nb = b_hi - b_lo;
  const int64_t kb0 = b_lo + nb * sub / p.spc, kb1 = b_lo + nb * (sub + 1) / p.spc;
  const int64_t v0 = static_cast<int64_t>(rt) * kGRows, d0 = static_cast<int64_t>(dt) * (64 * NBF);
  const Opnd A = make_opnd(p.P, p.N64, v0, p.Tv, 1, wave, lane);
  const Opnd B = make_opnd(p.wt, p.N64, d0, p.D, 1, wave, lane);
  f32x16_t acc[4][NBF];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NBF; ++j) acc[i][j] = f32x16_t{};
  auto hook = [&](int kb, char* stage) {
    const int64_t kbase = (kb0 + kb) * kGK;
    if (kbase < lo || kbase + kGK > hi) {  // a block shared with the neighbouring chunk
      mask_units(stage, kbase, lo, hi);
      __syncthreads();
    }
  };
  gemm_loop(acc, A, B, kb0 * kGK, static_cast<int>(kb1 - kb0), lds, wave, lane, hook);

  float* dst = p.out_part + static_cast<int64_t>(split) * p.Tv * p.D;
  // (a uniform branch: a select per element kept both forms of every value live)
  auto store = [&](auto round_tag) {
    constexpr bool RND = decltype(round_tag)::value;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t t = v0 + 128 * wa + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
        if (t >= p.Tv) continue;
#pragma unroll
        for (int j = 0; j < NBF; ++j) {
          const int64_t d = d0 + 32 * NBF * wb + 32 * j + u;
          if (d < p.D) dst[t * p.D + d] = RND ? round_bf16(acc[i][j][v]) : acc[i][j][v];
        }
      }
    }
  };
  if (MAYROUND && p.round_out)
    store(std::true_type{});
  else
    store(std::false_type{});
}
template <int NBF, bool MAYROUND = false>
__global__ __launch_bounds__(kGThreads) void tiled_write_kernel(TWriteParams p) {
  write_body<NBF, MAYROUND>(p, blockIdx.x);
}
// Several independent products in one launch (the backward's five gradient
// contractions): group i owns workgroups [start[i], start[i + 1]), each
// range a multiple of 8 so that the workgroup -> XCD mapping is the
// single-product one.
constexpr int kWriteBatch = 5;
struct TWriteBatch {
  TWriteParams p[kWriteBatch];
  int start[kWriteBatch + 1];
  int n;
};
template <int NBF>
__global__ __launch_bounds__(kGThreads) void tiled_write_batch_kernel(TWriteBatch b) {
  int i = 0;
  for (int k = 1; k < b.n; ++k) i += static_cast<int>(blockIdx.x) >= b.start[k] ? 1 : 0;
  write_body<NBF, true>(b.p[i], static_cast<int>(blockIdx.x) - b.start[i]);
}

// per-token sums of the gate kernel's partials, in a fixed order:
// sum[t] = sum over s of part[s][t] (sum gate, sum intensity, active count).
// 64 tokens per workgroup, four partial groups s = g mod 4 per token with
// eight loads in flight each, combined in LDS.
__global__ __launch_bounds__(256) void tiled_tok_sum_kernel(const float* __restrict__ part, float* __restrict__ sum,
                                                            int64_t Tv, int S) {
  __shared__ float4 red[4][64];
  const int c = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + c;
  const int64_t tl = t < Tv ? t : Tv - 1;
  float4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = float4{0.f, 0.f, 0.f, 0.f};
  int s = grp;
  for (; s + 28 < S; s += 32) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 q = *reinterpret_cast<const float4*>(part + (static_cast<int64_t>(s + 4 * k) * Tv + tl) * 4);
      acc[k].x += q.x;
      acc[k].y += q.y;
      acc[k].z += q.z;
    }
  }
  for (; s < S; s += 4) {
    const float4 q = *reinterpret_cast<const float4*>(part + (static_cast<int64_t>(s) * Tv + tl) * 4);
    acc[0].x += q.x;
    acc[0].y += q.y;
    acc[0].z += q.z;
  }
#pragma unroll
  for (int k = 1; k < 8; ++k) {
    acc[0].x += acc[k].x;
    acc[0].y += acc[k].y;
    acc[0].z += acc[k].z;
  }
  red[grp][c] = acc[0];
  __syncthreads();
  if (grp == 0 && t < Tv) {
    float4 r = red[0][c];
#pragma unroll
    for (int g = 1; g < 4; ++g) {
      r.x += red[g][c].x;
      r.y += red[g][c].y;
      r.z += red[g][c].z;
    }
    r.w = 0.f;
    *reinterpret_cast<float4*>(sum + t * 4) = r;
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct TGeo {
  int64_t Tv, N, N64, cs;
  int nc, RT, CT, DT, spc, S;
};

int64_t al256(int64_t b) { return (b + 255) & ~static_cast<int64_t>(255); }

TGeo tgeo(const srw_desc_t& d) {
  TGeo g{};
  g.Tv = d.T * d.n_routes;
  g.N = d.n_units;
  g.N64 = (g.N + kNAlign - 1) / kNAlign * kNAlign;
  g.cs = d.chunk_size > 0 && d.chunk_size < d.n_units ? d.chunk_size : d.n_units;
  g.nc = static_cast<int>((g.N + g.cs - 1) / g.cs);
  g.RT = static_cast<int>((g.Tv + kGRows - 1) / kGRows);
  g.CT = static_cast<int>((g.N + kGRows - 1) / kGRows);
  g.DT = static_cast<int>((d.d_model + kGRows - 1) / kGRows);
  // splits per chunk of the write GEMM: enough workgroups for 256 CUs, every
  // split at least one k block
  int64_t min_blocks = INT64_MAX;
  for (int c = 0; c < g.nc; ++c) {
    const int64_t lo = c * g.cs, hi = (c + 1) * g.cs < g.N ? (c + 1) * g.cs : g.N;
    const int64_t nb = (hi + kGK - 1) / kGK - lo / kGK;
    min_blocks = nb < min_blocks ? nb : min_blocks;
  }
  const int64_t per_split = static_cast<int64_t>(g.RT) * g.DT * g.nc;
  int64_t spc = (512 + per_split - 1) / per_split;
  spc = spc < 1 ? 1 : spc;
  spc = spc > min_blocks ? min_blocks : spc;
  g.spc = static_cast<int>(spc);
  g.S = g.nc * g.spc;
  return g;
}

struct TLayout {
  size_t wt, P, mom, tau, out_part, tok_part, tok_sum, uni, list, glist, cstart, G, total;
};

// sparse skip at prefill sizes: the gathered GEMMs' widths (D = 256 F; a
// wider D would not keep the gather kernel's fragments in 256 registers),
// R and W rows addressed by 32-bit byte offsets
bool sparse_width_ok(int64_t D) { return D == 256 || D == 512 || D == 1024; }
bool tiled_sparse(const srw_desc_t& d) {
  return (d.flags & SRW_FLAG_SPARSE_SKIP) && !(d.flags & SRW_FLAG_GATE_OUT) && sparse_width_ok(d.d_model) &&
         d.n_units * d.d_model * 2 < (int64_t(1) << 32);
}

TLayout tlayout(const srw_desc_t& d, const TGeo& g) {
  TLayout l{};
  size_t off = 0;
  l.wt = off;
  off += al256(d.d_model * g.N64 * 2);
  l.P = off;
  off += al256(g.Tv * g.N64 * 2);
  l.mom = off;
  off += al256(static_cast<int64_t>(2 * g.CT) * g.Tv * 2 * 4);
  l.tau = off;
  off += al256(g.Tv * 4);
  l.out_part = off;
  off += al256(static_cast<int64_t>(g.S) * g.Tv * d.d_model * 4);
  l.tok_part = off;
  off += al256(static_cast<int64_t>(2 * g.CT) * g.Tv * 4 * 4);
  l.tok_sum = off;
  off += al256(g.Tv * 4 * 4);
  // sparse skip: per 32-token tile the union words, the unit list and the
  // units' slots in G, the chunk starts, and G (256 CT slots of 32 gates)
  l.uni = l.list = l.glist = l.cstart = l.G = off;
  if (tiled_sparse(d)) {
    const int64_t tt = (g.Tv + 31) / 32, w32 = (g.N + 31) / 32;
    l.list = l.uni + al256(tt * w32 * 4);
    l.glist = l.list + al256(tt * g.N * 4);
    l.cstart = l.glist + al256(tt * g.N * 4);
    l.G = l.cstart + al256(tt * (g.nc + 1) * 4);
    off = l.G + al256(tt * (static_cast<int64_t>(g.CT) * 256) * 32 * 2);
  }
  l.total = off;
  return l;
}

hipError_t set_lds(const void* fn, int bytes = kGemmLds) {
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

}  // namespace

// The operand loaders keep each lane's byte offset within a 256-row tile in
// 32 bits: 256 rows of ld bf16 elements must stay below 4 GiB (ld = N or T
// padded to 64 for the stored [., N64] / [., T64] arrays).
static bool tile_offsets_fit(int64_t ld) { return 256 * ((ld + kNAlign - 1) / kNAlign * kNAlign) * 2 < (int64_t(1) << 32); }

bool tiled_supports(const srw_desc_t& d) {
  if (d.dtype != SRW_BF16 || d.gate != SRW_GATE_V41) return false;
  if (!tile_offsets_fit(d.n_units)) return false;
  if (d.stats_mode != SRW_STATS_ONEPASS && d.stats_mode != SRW_STATS_CENTERED) return false;
  // SRW_FLAG_SPARSE_SKIP: d_model = 256, 512 or 1024 takes the sparse-skip
  // kernels (mark, list, gathered GEMMs); other widths run dense
  if (d.flags & (SRW_FLAG_DIAG | SRW_FLAG_EMULATE | SRW_FLAG_NO_FAST)) return false;
  if (d.n_routes != 1 && d.n_routes != 2) return false;
  if (d.d_model % kNAlign != 0 || d.d_route % kNAlign != 0) return false;
  return true;
}

size_t tiled_workspace_bytes(const srw_desc_t& d) { return tlayout(d, tgeo(d)).total; }

bool tiled_runs_sparse(const srw_desc_t& d) { return tiled_sparse(d); }

// Sparse skip after the dense score GEMM and tau: mark, list, the gathered
// GEMMs, then the token sums and the finalize as on the dense path.
hipError_t tiled_sparse_rest(const LaunchArgs& a, const TGeo& g, const TLayout& l) {
  const srw_desc_t& d = a.d;
  const int D = static_cast<int>(d.d_model);
  const uint16_t* S = reinterpret_cast<const uint16_t*>(a.ws + l.P);
  const float* tau = reinterpret_cast<const float*>(a.ws + l.tau);
  float* out_part = reinterpret_cast<float*>(a.ws + l.out_part);
  float* tok_part = reinterpret_cast<float*>(a.ws + l.tok_part);
  float* tok_sum = reinterpret_cast<float*>(a.ws + l.tok_sum);
  uint32_t* uni = reinterpret_cast<uint32_t*>(a.ws + l.uni);
  int32_t* list = reinterpret_cast<int32_t*>(a.ws + l.list);
  int32_t* glist = reinterpret_cast<int32_t*>(a.ws + l.glist);
  int32_t* cstart = reinterpret_cast<int32_t*>(a.ws + l.cstart);
  uint16_t* G = reinterpret_cast<uint16_t*>(a.ws + l.G);
  const int64_t TT32 = (g.Tv + 31) / 32, W32 = (g.N + 31) / 32, GS = static_cast<int64_t>(g.CT) * 256;
  const float exp_scale = -d.sharpness * 1.4426950408889634f;
  hipError_t e;
  SpMarkParams mp{};
  mp.S = S;
  mp.tau = tau;
  mp.tok_part = tok_part;
  mp.mask32 = reinterpret_cast<uint32_t*>(a.o.pass_mask);
  mp.uni = uni;
  mp.G = G;
  mp.mask_words32 = 2 * a.words;
  mp.W32 = W32;
  mp.GS = GS;
  mp.Tv = g.Tv;
  mp.N = g.N;
  mp.N64 = g.N64;
  mp.CT = g.CT;
  mp.gp = a.gp;
  mp.exp_scale = exp_scale;
  const int64_t sgroups = (2 * g.CT + 3) / 4;
  hipLaunchKernelGGL(sp_mark_kernel, dim3(static_cast<unsigned>(TT32 * sgroups)), dim3(256), 0, a.stream, mp);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(tiled_tok_sum_kernel, dim3(static_cast<unsigned>((g.Tv + 63) / 64)), dim3(256), 0, a.stream,
                     tok_part, tok_sum, g.Tv, 2 * g.CT);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(sp_list_kernel, dim3(static_cast<unsigned>(TT32)), dim3(256), 0, a.stream, uni, W32, g.N, g.cs,
                     g.nc, list, glist, cstart);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  SpGatherParams sp{};
  sp.x = static_cast<const uint16_t*>(a.in.x);
  sp.read = static_cast<const uint16_t*>(a.in.read);
  sp.write = static_cast<const uint16_t*>(a.in.write);
  sp.G = G;
  sp.list = list;
  sp.glist = glist;
  sp.cstart = cstart;
  sp.out_part = out_part;
  sp.Tv = g.Tv;
  sp.N = g.N;
  sp.GS = GS;
  sp.routes = d.n_routes;
  sp.nc = g.nc;
  sp.TT32 = static_cast<int>(TT32);
  const dim3 grid_g(static_cast<unsigned>(TT32 * g.nc));  // (chunk, tile), chunk-major
  dominant_kernel_begin(a.stream);
  switch (D / 256) {
    case 1: hipLaunchKernelGGL(sp_gather_kernel<1>, grid_g, dim3(kSpThreads), 0, a.stream, sp); break;
    case 2: hipLaunchKernelGGL(sp_gather_kernel<2>, grid_g, dim3(kSpThreads), 0, a.stream, sp); break;
    default: hipLaunchKernelGGL(sp_gather_kernel<4>, grid_g, dim3(kSpThreads), 0, a.stream, sp); break;
  }
  dominant_kernel_end(a.stream);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  FinalizeArgs f{};
  f.out_part = out_part;
  f.tok_part = tok_sum;
  f.out = static_cast<uint16_t*>(a.o.out);
  f.gate_sum = a.o.gate_sum;
  f.den = a.o.den;
  f.n_active = a.o.n_active;
  f.T = g.Tv;
  f.D = D;
  f.S = g.nc;  // one partial per reference chunk
  f.spc = 1;
  f.S_tok = 1;
  f.tps = 4;
  f.scale = d.scale;
  f.gp = a.gp;
  f.exp_scale = exp_scale;
  return launch_finalize(f, a.stream);
}

hipError_t tiled_forward(const LaunchArgs& a) {
  const srw_desc_t& d = a.d;
  const TGeo g = tgeo(d);
  const TLayout l = tlayout(d, g);
  uint16_t* wt = reinterpret_cast<uint16_t*>(a.ws + l.wt);
  uint16_t* P = reinterpret_cast<uint16_t*>(a.ws + l.P);
  float* mom = reinterpret_cast<float*>(a.ws + l.mom);
  float* tau = reinterpret_cast<float*>(a.ws + l.tau);
  float* out_part = reinterpret_cast<float*>(a.ws + l.out_part);
  float* tok_part = reinterpret_cast<float*>(a.ws + l.tok_part);
  float* tok_sum = reinterpret_cast<float*>(a.ws + l.tok_sum);
  const int D = static_cast<int>(d.d_model);
  hipError_t e;
  static_assert(kGemmLds <= 160 * 1024, "LDS per workgroup");
  for (const void* fn : {reinterpret_cast<const void*>(tiled_stats_kernel),
                         reinterpret_cast<const void*>(tiled_gate_kernel<false>),
                         reinterpret_cast<const void*>(tiled_gate_kernel<false, true>),
                         reinterpret_cast<const void*>(tiled_write_kernel<4>)})
    if ((e = set_lds(fn)) != hipSuccess) return e;

  if (!(d.flags & SRW_FLAG_POOL_CACHED) && !tiled_sparse(d)) {  // (the sparse path gathers W's rows)
    const dim3 grid_p(static_cast<unsigned>(g.N64 / 64), static_cast<unsigned>((D + 63) / 64));
    hipLaunchKernelGGL(pack_wt_kernel, grid_p, dim3(256), 0, a.stream, static_cast<const uint16_t*>(a.in.write), wt,
                       g.N, g.N64, D);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  const unsigned grid_rc = static_cast<unsigned>(8 * g.RT * ((g.CT + 7) / 8));
  TStatsParams sp{};
  sp.h = static_cast<const uint16_t*>(a.in.h);
  sp.emb = static_cast<const uint16_t*>(a.in.emb);
  sp.S = P;
  sp.mom = mom;
  sp.Tv = g.Tv;
  sp.N = g.N;
  sp.N64 = g.N64;
  sp.dr = d.d_route;
  sp.RT = g.RT;
  sp.CT = g.CT;
  sp.centred = d.stats_mode == SRW_STATS_CENTERED;
  hipLaunchKernelGGL(tiled_stats_kernel, dim3(grid_rc), dim3(kGThreads), kGemmLds, a.stream, sp);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  // tau per row from the 2 CT partials of 128 units (centred: merged by
  // Chan's formula, no second pass over the stored scores)
  if ((e = launch_tau(mom, a.in.tau_offset, tau, g.Tv, 2 * g.CT, g.N, 2, nullptr,
                      d.stats_mode == SRW_STATS_CENTERED ? kTauChan : kTauOnePass, a.stream, nullptr, 128)) !=
      hipSuccess)
    return e;

  if (tiled_sparse(d)) return tiled_sparse_rest(a, g, l);

  TGateParams gp{};
  gp.x = static_cast<const uint16_t*>(a.in.x);
  gp.read = static_cast<const uint16_t*>(a.in.read);
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
  gp.RT = g.RT;
  gp.CT = g.CT;
  gp.gp = a.gp;
  gp.exp_scale = -d.sharpness * 1.4426950408889634f;
  dominant_kernel_begin(a.stream);
  if (gp.G)
    hipLaunchKernelGGL((tiled_gate_kernel<false, true>), dim3(grid_rc), dim3(kGThreads), kGemmLds, a.stream, gp);
  else
    hipLaunchKernelGGL(tiled_gate_kernel<false>, dim3(grid_rc), dim3(kGThreads), kGemmLds, a.stream, gp);
  dominant_kernel_end(a.stream);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  TWriteParams wp{};
  wp.P = P;
  wp.wt = wt;
  wp.out_part = out_part;
  wp.Tv = g.Tv;
  wp.N = g.N;
  wp.N64 = g.N64;
  wp.D = D;
  wp.cs = g.cs;
  wp.nc = g.nc;
  wp.spc = g.spc;
  wp.S = g.S;
  wp.RT = g.RT;
  wp.DT = g.DT;
  const unsigned grid_w = static_cast<unsigned>(8 * g.DT * ((static_cast<int64_t>(g.RT) * g.S + 7) / 8));
  hipLaunchKernelGGL(tiled_write_kernel<4>, dim3(grid_w), dim3(kGThreads), kGemmLds, a.stream, wp);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  hipLaunchKernelGGL(tiled_tok_sum_kernel, dim3(static_cast<unsigned>((g.Tv + 63) / 64)), dim3(256), 0, a.stream,
                     tok_part, tok_sum, g.Tv, 2 * g.CT);
  if ((e = hipGetLastError()) != hipSuccess) return e;

  FinalizeArgs f{};
  f.out_part = out_part;
  f.tok_part = tok_sum;
  f.out = static_cast<uint16_t*>(a.o.out);
  f.gate_sum = a.o.gate_sum;
  f.den = a.o.den;
  f.n_active = a.o.n_active;
  f.T = g.Tv;
  f.D = D;
  f.S = g.S;
  f.spc = g.spc;
  f.S_tok = 1;
  f.tps = 4;
  f.scale = d.scale;
  f.gp = a.gp;
  f.exp_scale = -d.sharpness * 1.4426950408889634f;
  return launch_finalize(f, a.stream);
}

// ===========================================================================
// Backward (VJP) of fused_gate_srw for one route: the gradients of
// <d_out, out> + d_lb * score_lb + d_pen * dead_penalty (the outputs the
// reference's training loss uses, scripts/train_jax.py:586-603) with respect
// to x, h, emb, tau_offset, read and write.  The forward's scores, gates and
// products are recomputed (the reference checkpoints both scans, v41:434,
// 489); every [T, N] intermediate lives in the workspace in bf16 (the
// derivative of the gate in fp32), and the six contractions run on the same
// tiled MFMA main loop as the forward:
//   dP  = draw . W^T          (epilogue: the gate derivative -> dm, d(xr))
//   dW  = P^T . draw,  dR = d(xr)^T . x,  dE = ds^T . h       (K = tokens)
//   dx  = d(xr) . R,   dh = ds . E                             (K = units)
// ===========================================================================
namespace {

// per-token mean, variance, std + 1e-8 and tau from the moment partials
// (same expressions as srw_tau_kernel, v41:461-464)
__global__ __launch_bounds__(256) void bwd_token_stats_kernel(const float* __restrict__ mom, int S_st, int64_t T,
                                                              int64_t N, const float* __restrict__ tau_off,
                                                              float* __restrict__ mean, float* __restrict__ var,
                                                              float* __restrict__ sdev, float* __restrict__ tau) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float a = 0.f, b = 0.f;
  for (int s = lane; s < S_st; s += 64) {
    a += mom[(static_cast<int64_t>(s) * T + t) * 2];
    b += mom[(static_cast<int64_t>(s) * T + t) * 2 + 1];
  }
  a = wave_sum(a);
  b = wave_sum(b);
  if (lane == 0) {
    const float fN = static_cast<float>(N);
    const float mu = a / fN;
    const float v = b / fN - __fmul_rn(mu, mu);
    const float sd = sqrtf(v) + 1e-8f;
    mean[t] = mu;
    var[t] = v;
    sdev[t] = sd;
    tau[t] = mu + __fmul_rn(tau_off[t], sd);
  }
}

// draw = bf16(d_out * scale) / den as bf16 (the cotangent of the chunk dots),
// and the den term dden = -sum_d dq * (raw / den) / den where den = max(sum
// intensity, 1) is differentiable (v41:584-585); raw / den from the forward's
// out.  dsc[t] = sum_d d_out * out / scale: the row's share of the gradient
// of the scale the caller multiplies out by (v41:1044-1053, 1175).
__global__ __launch_bounds__(256) void bwd_prep_kernel(const float* __restrict__ d_out,
                                                       const uint16_t* __restrict__ out,
                                                       const float* __restrict__ zsums, int zs_stride, float scale,
                                                       int D, uint16_t* __restrict__ draw,
                                                       float* __restrict__ dden, float* __restrict__ dsc) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const float zsum = zsums[t * zs_stride];  // sum intensity of the row
  const float den = fmaxf(zsum, 1.0f);
  float acc = 0.f, acc_s = 0.f;
  for (int d = threadIdx.x; d < D; d += 256) {
    const float g = d_out[t * D + d];
    const float dq = round_bf16(g * scale);
    const float o = bf16_to_f32(out[t * D + d]) / scale;
    acc += dq * o;
    acc_s += g * o;
    draw[t * D + d] = f32_to_bf16_bits(dq / den);
  }
  acc = block_sum<256>(acc, red);
  if (threadIdx.x == 0) dden[t] = zsum > 1.0f ? -acc / den : 0.f;
  acc_s = block_sum<256>(acc_s, red);
  if (threadIdx.x == 0) dsc[t] = acc_s;
}

// out[0] = sum of v[0 .. n) in one workgroup (a fixed order: deterministic).
__global__ __launch_bounds__(256) void bwd_total_kernel(const float* __restrict__ v, int64_t n,
                                                        float* __restrict__ out) {
  __shared__ float red[4];
  float acc = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 256) acc += v[i];
  acc = block_sum<256>(acc, red);
  if (threadIdx.x == 0) out[0] = acc;
}

// Plain MFMA GEMM, bf16 out: C[t][n] = A[n, :] . B[t / div, :] over K for a
// 256-unit x 256-row tile (A = units, B = rows), stored as [rows, N64] bf16
// (the dot outputs the reference rounds to bf16: x.r, v41:517; the dP
// transpose of the chunk dots, v41:518).  Units past N hold values of the
// clamped last row: every consumer masks them.
struct TStoreParams {
  const uint16_t* A;  // [N, K]
  const uint16_t* B;  // [rows_b, K]
  uint16_t* C;        // [rows, N64]
  int64_t rows, rows_b, N, N64, K;
  int div, RT, CT;
};

__global__ __launch_bounds__(kGThreads) void tiled_store_kernel(TStoreParams p) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wa = wave >> 1, wb = wave & 1, u = lane & 31, h = lane >> 5;
  int rt, ct;
  if (!tile_of(p.RT, p.CT, rt, ct)) return;
  const int64_t u0 = static_cast<int64_t>(ct) * kGRows, v0 = static_cast<int64_t>(rt) * kGRows;
  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};
  {
    const Opnd A = make_opnd(p.A, p.K, u0, p.N, 1, wave, lane);
    const Opnd B = make_opnd(p.B, p.K, v0, p.rows, p.div, wave, lane);
    gemm_loop(acc, A, B, 0, static_cast<int>(p.K / kGK), lds, wave, lane, NoHook{});
  }
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t t = v0 + 128 * wb + 32 * j + u;
    if (t >= p.rows) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int v = 0; v < 16; v += 4) {
        const int64_t n0 = u0 + 128 * wa + 32 * i + 8 * (v >> 2) + 4 * h;
        if (n0 < p.N64)
          *reinterpret_cast<u32x2_t*>(p.C + t * p.N64 + n0) =
              u32x2_t{pack_bf16(acc[i][j][v], acc[i][j][v + 1]), pack_bf16(acc[i][j][v + 2], acc[i][j][v + 3])};
      }
    }
  }
}

// Elementwise passes over 64-row x 64-unit tiles of the [rows, N64] arrays:
// thread (rp, q) = (tid / 8, tid % 8) owns rows 2 rp, 2 rp + 1 (one token's
// two routes when paired) and units 8 q .. 8 q + 7; transposed copies go
// through an LDS tile and leave as 16-byte row pieces.
constexpr int kTile = 64;

struct ElemTile {
  int64_t v0, n0;  // first row, first unit
  int rp, q;
};
__device__ inline ElemTile elem_tile() {
  return ElemTile{static_cast<int64_t>(blockIdx.y) * kTile, static_cast<int64_t>(blockIdx.x) * kTile,
                  static_cast<int>(threadIdx.x >> 3), static_cast<int>(threadIdx.x & 7)};
}
__device__ inline void load8_bf16(const uint16_t* p, float (&f)[8]) {
  const u32x4_t w = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = lo_f32(w[k]);
    f[2 * k + 1] = hi_f32(w[k]);
  }
}
__device__ inline void store8_bf16(uint16_t* p, const float (&f)[8]) {
  *reinterpret_cast<u32x4_t*>(p) = u32x4_t{pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]),
                                           pack_bf16(f[6], f[7])};
}
// sum over the 8 threads of one row pair (consecutive lanes)
__device__ inline float rowsum8(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  return v;
}
// tile[r][c] (bf16 bits, rows = tile rows) -> dst [cols, ld]: column c of the
// tile is dst row n0 + c, rows r0 .. r0 + nr - 1 (nr a multiple of 8)
__device__ inline void store_transposed(const uint16_t (*tile)[kTile + 8], int nr, uint16_t* dst, int64_t ld,
                                        int64_t n0, int64_t r0, int64_t ncols) {
  for (int idx = threadIdx.x; idx < kTile * (nr / 8); idx += 256) {
    const int c = idx / (nr / 8), k = idx % (nr / 8);
    if (n0 + c >= ncols) continue;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = static_cast<uint32_t>(tile[8 * k + 2 * e][c]) | (static_cast<uint32_t>(tile[8 * k + 2 * e + 1][c]) << 16);
    *reinterpret_cast<u32x4_t*>(dst + (n0 + c) * ld + r0 + 8 * k) = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

struct ElemParams {
  const uint16_t* S;      // [Tv, N64] bf16 scores
  const uint16_t* XR;     // [T, N64] bf16 x.r per token
  const uint16_t* DP;     // [Tv, N64] bf16 dP (E2)
  const float* tau;       // [Tv]
  const float* dden;      // [Tv] (E2)
  uint16_t* PT;           // [N64, Tv64] P^T (E1)
  float* inten_part;      // [N64 / 64][Tv] sum intensity partials (E1)
  float* psum;            // [Tv64 / 64][N64] column sums of s (E1)
  float* pmax;            // [Tv64 / 64][N64] column maxima of the gate (E1)
  uint16_t* DXR;          // [T, N64] d(xr) per token (E2)
  uint16_t* DXRT;         // [N64, T64] (E2)
  float* dm_part;         // [N64 / 64][Tv] (E2)
  float* dmz_part;        // [N64 / 64][Tv] sums of dm z (E2, the v4.0.1 gate)
  const float* sdev;      // [Tv] s_std (the v4.0.1 gate's z scale)
  int64_t Tv, N, N64, Tv64, T64;
  int routes;
  GateParams gp;
  float exp_scale, sharp;
};

// E1: the forward's gates from the stored scores and x.r: P^T = bf16(bf16(g) *
// xr)^T (v41:516-518), per-row sum intensity partials (den, v41:527, 584),
// per-unit column sums of s and maxima of the gate (score_lb / dead penalty,
// v41:445, 543)
// GL: the v4.0.1 gate (v401:303-310): the forward kernels' z Phi(z) and, for
// den = max(sum gate, 1) (v401:340), per-row sums of the gate.
template <bool GL>
__global__ __launch_bounds__(256) void bwd_fwd_elem_kernel(ElemParams p) {
  __shared__ uint16_t tile[kTile][kTile + 8];
  __shared__ float cs[32][kTile + 1], cm[32][kTile + 1];
  const ElemTile et = elem_tile();
  const float c_exp = p.exp_scale, eps = p.gp.eps, maxi = p.gp.maxi;
  float colsum[8] = {}, colmax[8] = {};
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int r = 2 * et.rp + rr;
    const int64_t v = et.v0 + r;
    const int64_t n = et.n0 + 8 * et.q;
    const bool row_ok = v < p.Tv;
    const int64_t vl = row_ok ? v : p.Tv - 1;
    float s[8], x[8], pr[8];
    load8_bf16(p.S + vl * p.N64 + n, s);
    load8_bf16(p.XR + (vl / p.routes) * p.N64 + n, x);
    const float tau_thr = p.tau[vl] + p.gp.thr;
    const float k_exp = -tau_thr * c_exp, tau_cut = tau_thr + p.gp.cut;
    const float istd = GL ? 1.0f / p.sdev[vl] : 0.f;
    float isum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool ok = row_ok && n + e < p.N;
      float g, it;
      if constexpr (GL) {
        float zp;
        g = gelu_gate(s[e], p.tau[vl], istd, zp);
        it = g;  // the row sum is the gate sum
      } else {
        const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(fmaf(s[e], c_exp, k_exp)));
        it = eps + __builtin_amdgcn_fmed3f(s[e] - tau_cut, 0.0f, maxi);
        g = act * it;
      }
      pr[e] = ok ? round_bf16(g) * x[e] : 0.f;  // bf16 product, rounded by the packing below
      isum += ok ? it : 0.f;
      colsum[e] += ok ? s[e] : 0.f;
      colmax[e] = fmaxf(colmax[e], ok ? g : 0.f);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t w = pack_bf16(pr[2 * k], pr[2 * k + 1]);
      tile[r][8 * et.q + 2 * k] = static_cast<uint16_t>(w);
      tile[r][8 * et.q + 2 * k + 1] = static_cast<uint16_t>(w >> 16);
    }
    isum = rowsum8(isum);
    if (et.q == 0 && row_ok) p.inten_part[static_cast<int64_t>(blockIdx.x) * p.Tv + v] = isum;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    cs[et.rp][8 * et.q + e] = colsum[e];
    cm[et.rp][8 * et.q + e] = colmax[e];
  }
  __syncthreads();
  if (threadIdx.x < kTile) {
    float a = 0.f, m = 0.f;
    for (int k = 0; k < 32; ++k) {
      a += cs[k][threadIdx.x];
      m = fmaxf(m, cm[k][threadIdx.x]);
    }
    p.psum[static_cast<int64_t>(blockIdx.y) * p.N64 + et.n0 + threadIdx.x] = a;
    p.pmax[static_cast<int64_t>(blockIdx.y) * p.N64 + et.n0 + threadIdx.x] = m;
  }
  store_transposed(tile, kTile, p.PT, p.Tv64, et.n0, et.v0, p.N64);
}

// The gate derivative of one element (v41:506-518) from its bf16 score s,
// x.r and dP: d(gate_bf) and d(xr) from the bf16 product, then through act *
// intensity, the cutoff / cap clamps and the den term dden to dm, the
// cotangent of the margin m = s - tau - thr.  Written once, without
// contraction, so that bwd_gate_elem_kernel's row sums of dm and
// bwd_ds_elem_kernel's recomputed dm are the same values.
struct GateGrad {
  float dm, dx, gb;  // gb: the bf16 gate (v41:516)
};
__device__ inline GateGrad gate_grad(float s, float x, float dp, float tau, float dden, const GateParams& gp,
                                     float exp_scale, float sharp) {
#pragma clang fp contract(off)
  const float m = (s - tau) - gp.thr;
  const float act = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(m * exp_scale));
  const float am = fmaxf(m - gp.cut, 0.0f);
  const float it = gp.eps + fminf(am, gp.maxi);
  const float gb = round_bf16(act * it);
  const float dgb = round_bf16(dp * x);  // d(gate_bf): bf16 multiply transpose
  const float dx = round_bf16(dp * gb);  // d(xr)
  const float dit = dgb * act + dden;
  const float dam = am < gp.maxi ? dit : 0.f;
  const float dm = (m - gp.cut > 0.f ? dam : 0.f) + dgb * it * sharp * act * (1.0f - act);
  return GateGrad{dm, dx, gb};
}

// Phi(z) = 0.5 (1 + erf(z / sqrt 2)) for z >= 0, erf by Abramowitz & Stegun
// 7.1.26 (the forward kernels' gelu_gate evaluates the same expression).
__device__ inline float gelu_cdf_pos(float z) {
  const float x = z * 0.7071067811865476f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, x, 1.0f));
  float q = fmaf(1.061405429f, t, -1.453152027f);
  q = fmaf(q, t, 1.421413741f);
  q = fmaf(q, t, -0.284496736f);
  q = fmaf(q, t, 0.254829592f);
  return 0.5f * (1.0f + (1.0f - q * t * __builtin_amdgcn_exp2f(-x * x * 1.4426950408889634f)));
}

// The v4.0.1 gate's derivative of one element (v401:303-309): z = (s - tau) /
// s_std, gate = z Phi(z) for z > 0 (the forward's gelu_gate, so that P and
// the gates here are the forward's), d(gate_bf) and d(xr) from the bf16
// product, the den term (den = max(sum gate, 1), v401:340: every gate's
// cotangent gains dden), then dz = dgate (Phi(z) + z phi(z)) for z > 0, phi
// the normal density.  dm: the cotangent of s - tau, dz / s_std; dmz = dm z
// (the s_std chain: d s_std = -sum dm z).
struct GateGradGl {
  float dm, dmz, dx, gb;
};
__device__ inline GateGradGl gate_grad_gl(float s, float x, float dp, float tau, float istd, float dden) {
#pragma clang fp contract(off)
  float zp;
  const float g = gelu_gate(s, tau, istd, zp);
  const float z = (s - tau) * istd;
  const float gb = round_bf16(g);
  const float dgb = round_bf16(dp * x);  // d(gate_bf): bf16 multiply transpose
  const float dx = round_bf16(dp * gb);  // d(xr)
  const float dg = dgb + dden;
  const float pdf = 0.3989422804014327f * __builtin_amdgcn_exp2f(-0.5f * z * z * 1.4426950408889634f);
  const float dz = z > 0.f ? dg * (gelu_cdf_pos(z) + z * pdf) : 0.f;
  const float dm = dz * istd;
  return GateGradGl{dm, dm * z, dx, gb};
}

// E2: the gate derivative from the stored scores, x.r and dP: per-row sums of
// dm (the tau chain's input) and d(xr), summed over the routes of a token
// (the broadcast of x.r, v41:796-797) and stored in both layouts.  dm itself
// is not stored: the ds pass recomputes it from the same bf16 inputs (reading
// three bf16 arrays costs less than writing and reading an fp32 one).
// PT_OUT (the forward's den and unit statistics given, no E1 pass): also P^T
// = bf16(gate_bf * xr)^T (v41:516-518) from the same gate.
template <bool PT_OUT, bool GL = false>
__global__ __launch_bounds__(256) void bwd_gate_elem_kernel(ElemParams p) {
  __shared__ uint16_t tile[kTile][kTile + 8];
  __shared__ uint16_t ptile[PT_OUT ? kTile : 1][kTile + 8];
  const ElemTile et = elem_tile();
  const int64_t n = et.n0 + 8 * et.q;
  float dxs[2][8];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int r = 2 * et.rp + rr;
    const int64_t v = et.v0 + r;
    const bool row_ok = v < p.Tv;
    const int64_t vl = row_ok ? v : p.Tv - 1;
    float s[8], x[8], dp[8];
    load8_bf16(p.S + vl * p.N64 + n, s);
    load8_bf16(p.XR + (vl / p.routes) * p.N64 + n, x);
    load8_bf16(p.DP + vl * p.N64 + n, dp);
    const float tau = p.tau[vl], dden = p.dden[vl];
    const float istd = GL ? 1.0f / p.sdev[vl] : 0.f;
    float sdm = 0.f, sdmz = 0.f, pr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool ok = row_ok && n + e < p.N;
      float dm, dx, gb;
      if constexpr (GL) {
        const GateGradGl gg = gate_grad_gl(s[e], x[e], dp[e], tau, istd, dden);
        dm = gg.dm;
        dx = gg.dx;
        gb = gg.gb;
        sdmz += ok ? gg.dmz : 0.f;
      } else {
        const GateGrad gg = gate_grad(s[e], x[e], dp[e], tau, dden, p.gp, p.exp_scale, p.sharp);
        dm = gg.dm;
        dx = gg.dx;
        gb = gg.gb;
      }
      dxs[rr][e] = ok ? dx : 0.f;
      sdm += ok ? dm : 0.f;
      pr[e] = ok ? gb * x[e] : 0.f;  // bf16 product, rounded by the packing below
    }
    if constexpr (PT_OUT) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t w = pack_bf16(pr[2 * k], pr[2 * k + 1]);
        ptile[r][8 * et.q + 2 * k] = static_cast<uint16_t>(w);
        ptile[r][8 * et.q + 2 * k + 1] = static_cast<uint16_t>(w >> 16);
      }
    }
    sdm = rowsum8(sdm);
    if (et.q == 0 && row_ok) p.dm_part[static_cast<int64_t>(blockIdx.x) * p.Tv + v] = sdm;
    if constexpr (GL) {
      sdmz = rowsum8(sdmz);
      if (et.q == 0 && row_ok) p.dmz_part[static_cast<int64_t>(blockIdx.x) * p.Tv + v] = sdmz;
    }
  }
  // d(xr) per token: one row per route (single) or the pair's sum (paired)
  const int nt = p.routes == 2 ? kTile / 2 : kTile;  // tokens in this tile
  const int64_t t0 = p.routes == 2 ? et.v0 / 2 : et.v0;
  const int64_t T = p.Tv / p.routes;
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    if (p.routes == 2 && rr == 1) break;
    const int tr = p.routes == 2 ? et.rp : 2 * et.rp + rr;  // token row within the tile
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = p.routes == 2 ? dxs[0][e] + dxs[1][e] : dxs[rr][e];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t w = pack_bf16(o[2 * k], o[2 * k + 1]);
      tile[tr][8 * et.q + 2 * k] = static_cast<uint16_t>(w);
      tile[tr][8 * et.q + 2 * k + 1] = static_cast<uint16_t>(w >> 16);
    }
    if (t0 + tr < T) store8_bf16(p.DXR + (t0 + tr) * p.N64 + n, o);
  }
  __syncthreads();
  store_transposed(tile, nt, p.DXRT, p.T64, et.n0, t0, p.N64);
  if constexpr (PT_OUT) store_transposed(ptile, kTile, p.PT, p.Tv64, et.n0, et.v0, p.N64);
}

struct DsParams {
  const uint16_t* S;    // [Tv, N64]
  const uint16_t* XR;   // [T, N64]
  const uint16_t* DP;   // [Tv, N64]
  const float* tau;     // [Tv]
  const float* dden;    // [Tv]
  const float* alpha;   // [Tv]
  const float* beta;    // [Tv]
  const float* pn;      // [N64]
  const float* dead;    // [N64]
  const float* coef;    // {c0, c1}
  uint16_t* DS;         // [Tv, N64]
  uint16_t* DST;        // [N64, Tv64]
  const float* sdev;    // [Tv] s_std (the v4.0.1 gate)
  float d_pen;
  int64_t Tv, N, N64, Tv64;
  int routes;
  GateParams gp;
  float exp_scale, sharp;
};

// E3: ds = bf16(dm + alpha_v + beta_v s + (c0 + c1 pn[n] - d_pen [pn < 0] dead[n]) / Tv)
// (the tau chain, v41:461-464, and the per-unit score_lb / dead-penalty
// terms, v41:445-447, 543-552), zero past N; both layouts.  dm as in E2
// (gate_grad on the same bf16 inputs).
template <bool GL = false>
__global__ __launch_bounds__(256) void bwd_ds_elem_kernel(DsParams p) {
  __shared__ uint16_t tile[kTile][kTile + 8];
  const ElemTile et = elem_tile();
  const int64_t n = et.n0 + 8 * et.q;
  const float c0 = p.coef[0], c1 = p.coef[1];
  const float inv = 1.0f / static_cast<float>(p.Tv);
  float unit[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float pv = p.pn[n + e];
    unit[e] = (c0 + c1 * pv + (pv < 0.f ? -p.d_pen * p.dead[n + e] : 0.f)) * inv;
  }
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int r = 2 * et.rp + rr;
    const int64_t v = et.v0 + r;
    const bool row_ok = v < p.Tv;
    const int64_t vl = row_ok ? v : p.Tv - 1;
    float s[8], x[8], dp[8], o[8];
    load8_bf16(p.S + vl * p.N64 + n, s);
    load8_bf16(p.XR + (vl / p.routes) * p.N64 + n, x);
    load8_bf16(p.DP + vl * p.N64 + n, dp);
    const float a = p.alpha[vl], b = p.beta[vl], tau = p.tau[vl], dden = p.dden[vl];
    const float istd = GL ? 1.0f / p.sdev[vl] : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float dm;
      if constexpr (GL) dm = gate_grad_gl(s[e], x[e], dp[e], tau, istd, dden).dm;
      else dm = gate_grad(s[e], x[e], dp[e], tau, dden, p.gp, p.exp_scale, p.sharp).dm;
      o[e] = row_ok && n + e < p.N ? dm + a + b * s[e] + unit[e] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t w = pack_bf16(o[2 * k], o[2 * k + 1]);
      tile[r][8 * et.q + 2 * k] = static_cast<uint16_t>(w);
      tile[r][8 * et.q + 2 * k + 1] = static_cast<uint16_t>(w >> 16);
    }
    if (row_ok) store8_bf16(p.DS + v * p.N64 + n, o);
  }
  __syncthreads();
  store_transposed(tile, kTile, p.DST, p.Tv64, et.n0, et.v0, p.N64);
}

// sum[v] = sum over b of part[b][v] (fixed order), four partial groups per row
__global__ __launch_bounds__(256) void bwd_rowsum_kernel(const float* __restrict__ part, int nb, int64_t rows,
                                                         float* __restrict__ sum) {
  __shared__ float red[4][64];
  const int c = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t v = static_cast<int64_t>(blockIdx.x) * 64 + c;
  const int64_t vl = v < rows ? v : rows - 1;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  int b = grp;
  for (; b + 12 < nb; b += 16) {
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] += part[static_cast<int64_t>(b + 4 * k) * rows + vl];
  }
  for (; b < nb; b += 4) a[0] += part[static_cast<int64_t>(b) * rows + vl];
  red[grp][c] = (a[0] + a[1]) + (a[2] + a[3]);
  __syncthreads();
  if (grp == 0 && v < rows) sum[v] = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
}

// tau chain per token (v41:461-464): dtau = -sum_n dm; tau = mean + off * std,
// std = sqrt(E[s^2] - mean^2) + 1e-8.  Writes d tau_offset and the affine
// coefficients of the score gradient, ds = dm + alpha + beta * s (+ unit term)
// dmz_part (the v4.0.1 gate, else null): sums of dm z, z = (s - tau) / s_std;
// z's own dependence on s_std adds d s_std = -sum_n dm z (v401:304).  16 rows
// per workgroup, 16 partial groups per row (a block's partials are
// row-contiguous: 64-byte loads), combined in a fixed order.
constexpr int kTokRows = 16, kTokGroups = 16;
__global__ __launch_bounds__(256) void bwd_token_kernel(const float* __restrict__ dm_part,
                                                        const float* __restrict__ dmz_part, int S2, int64_t T,
                                                        int64_t N, const float* __restrict__ tau_off,
                                                        const float* __restrict__ mean, const float* __restrict__ var,
                                                        const float* __restrict__ sdev, float* __restrict__ dtau_off,
                                                        float* __restrict__ alpha, float* __restrict__ beta) {
  __shared__ float red[2][kTokGroups][kTokRows + 1];
  const int c = threadIdx.x % kTokRows, grp = threadIdx.x / kTokRows;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kTokRows + c;
  const int64_t tl = t < T ? t : T - 1;
  float a[2] = {0.f, 0.f}, z[2] = {0.f, 0.f};
  int b = grp;
  for (; b + kTokGroups < S2; b += 2 * kTokGroups) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      a[k] += dm_part[static_cast<int64_t>(b + kTokGroups * k) * T + tl];
      if (dmz_part) z[k] += dmz_part[static_cast<int64_t>(b + kTokGroups * k) * T + tl];
    }
  }
  for (; b < S2; b += kTokGroups) {
    a[0] += dm_part[static_cast<int64_t>(b) * T + tl];
    if (dmz_part) z[0] += dmz_part[static_cast<int64_t>(b) * T + tl];
  }
  red[0][grp][c] = a[0] + a[1];
  red[1][grp][c] = z[0] + z[1];
  __syncthreads();
  if (grp == 0 && t < T) {
    float sa = 0.f, sz = 0.f;
    for (int q = 0; q < kTokGroups; ++q) {
      sa += red[0][q][c];
      sz += red[1][q][c];
    }
    const float fN = static_cast<float>(N);
    const float dtau = -sa;
    dtau_off[t] = dtau * sdev[t];
    const float dstd = dtau * tau_off[t] - sz;
    const float dvar = dstd / (2.0f * sqrtf(var[t]));
    const float dmean = dtau - 2.0f * mean[t] * dvar;
    alpha[t] = dmean / fN;
    beta[t] = 2.0f * dvar / fN;
  }
}

// pn[n] = mean_t s, dead[n] = max_t gate < dead_threshold (v41:548), and
// per-block sums of pn, pn^2 over the units (v41:445-447)
__global__ __launch_bounds__(256) void bwd_unit_reduce_kernel(const float* __restrict__ psum,
                                                              const float* __restrict__ pmax, int TS, int64_t T,
                                                              int64_t N, int64_t N64, float dead_thr,
                                                              float* __restrict__ pn, float* __restrict__ dead,
                                                              float* __restrict__ blk) {
  __shared__ float red[4];
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  float sum = 0.f, gmax = 0.f;
  if (n < N64) {
    for (int s = 0; s < TS; ++s) {
      sum += psum[static_cast<int64_t>(s) * N64 + n];
      gmax = fmaxf(gmax, pmax[static_cast<int64_t>(s) * N64 + n]);
    }
  }
  const bool ok = n < N;
  const float m = ok ? sum / static_cast<float>(T) : 0.f;
  if (n < N64) {
    pn[n] = m;
    dead[n] = ok && gmax < dead_thr ? 1.0f : 0.0f;
  }
  const float a = block_sum<256>(m, red);
  const float b = block_sum<256>(m * m, red);
  if (threadIdx.x == 0) {
    blk[2 * blockIdx.x] = a;
    blk[2 * blockIdx.x + 1] = b;
  }
}

// The same from the forward's unit diagnostics (unit_diag[n][2] = sum of the
// unit's scores over the rows, its max gate): pn, dead and the block sums.
__global__ __launch_bounds__(256) void bwd_unit_from_diag_kernel(const float* __restrict__ ud, int64_t T, int64_t N,
                                                                 int64_t N64, float dead_thr, float* __restrict__ pn,
                                                                 float* __restrict__ dead, float* __restrict__ blk) {
  __shared__ float red[4];
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const bool ok = n < N;
  const float m = ok ? ud[n * SRW_UDIAG_COUNT + SRW_UDIAG_SCORE_SUM] / static_cast<float>(T) : 0.f;
  if (n < N64) {
    pn[n] = m;
    dead[n] = ok && ud[n * SRW_UDIAG_COUNT + SRW_UDIAG_GATE_MAX] < dead_thr ? 1.0f : 0.0f;
  }
  const float a = block_sum<256>(m, red);
  const float b = block_sum<256>(m * m, red);
  if (threadIdx.x == 0) {
    blk[2 * blockIdx.x] = a;
    blk[2 * blockIdx.x + 1] = b;
  }
}

// score_lb = var(pn) / (mean(pn)^2 + var(pn) + 1e-2) (v41:477-483): its
// derivative in pn[n] is c0 + c1 pn[n]; coef = {c0, c1} times d_lb
__global__ __launch_bounds__(256) void bwd_unit_coef_kernel(const float* __restrict__ blk, int nblk, int64_t N,
                                                            float d_lb, float* __restrict__ coef) {
  __shared__ float red[4];
  float a = 0.f, b = 0.f;
  for (int i = threadIdx.x; i < nblk; i += 256) {
    a += blk[2 * i];
    b += blk[2 * i + 1];
  }
  a = block_sum<256>(a, red);
  b = block_sum<256>(b, red);
  if (threadIdx.x == 0) {
    const float fN = static_cast<float>(N);
    const float ms = a / fN;
    const float vs = b / fN - ms * ms;
    const float Z = ms * ms + vs + 1e-2f;
    const float dvs = (ms * ms + 1e-2f) / (Z * Z);
    const float dms = -2.0f * ms * vs / (Z * Z);
    coef[0] = d_lb * (-dvs * 2.0f * ms / fN + dms / fN);
    coef[1] = d_lb * dvs * 2.0f / fN;
  }
}

// The v4.0.1 forward normalisation r_hat = r / (||r|| + 1e-8) of the read
// and write rows (v401:300-301), backwards, in place: grad holds d r_hat of
// each row on entry and d r = d r_hat / c - r (r . d r_hat) / (c^2 ||r||)
// (c = ||r|| + 1e-8) on exit.  One wave per row (four per workgroup), fp32
// from the bf16 rows.
__global__ __launch_bounds__(256) void bwd_norm_rows_kernel(const uint16_t* __restrict__ rows, float* __restrict__ grad,
                                                            int64_t N, int64_t D) {
  const int lane = threadIdx.x & 63;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  // four adjacent elements per lane and step (8- and 16-byte accesses; D is a
  // multiple of 64), rows of up to 1024 elements held between the two sweeps
  const uint2* r = reinterpret_cast<const uint2*>(rows + n * D);
  float4* g = reinterpret_cast<float4*>(grad + n * D);
  const int64_t D4 = D / 4;
  constexpr int kRegs = 4;
  float4 rv[kRegs], gv[kRegs];
  float ss = 0.f, dot = 0.f;
#pragma unroll
  for (int j = 0; j < kRegs; ++j) {
    const int64_t i = lane + 64 * j;
    if (i < D4) {
      const uint2 w = r[i];
      rv[j] = make_float4(lo_f32(w.x), hi_f32(w.x), lo_f32(w.y), hi_f32(w.y));
      gv[j] = g[i];
      ss += rv[j].x * rv[j].x + rv[j].y * rv[j].y + rv[j].z * rv[j].z + rv[j].w * rv[j].w;
      dot += rv[j].x * gv[j].x + rv[j].y * gv[j].y + rv[j].z * gv[j].z + rv[j].w * gv[j].w;
    }
  }
  for (int64_t i = lane + 64 * kRegs; i < D4; i += 64) {  // rows beyond 1024 elements
    const uint2 w = r[i];
    const float4 gg = g[i];
    const float a = lo_f32(w.x), b = hi_f32(w.x), c = lo_f32(w.y), d = hi_f32(w.y);
    ss += a * a + b * b + c * c + d * d;
    dot += a * gg.x + b * gg.y + c * gg.z + d * gg.w;
  }
  ss = wave_sum(ss);
  dot = wave_sum(dot);
  const float nrm = sqrtf(ss), c = nrm + 1e-8f;
  const float k = nrm > 0.f ? dot / (c * c * nrm) : 0.f;
#pragma unroll
  for (int j = 0; j < kRegs; ++j) {
    const int64_t i = lane + 64 * j;
    if (i < D4)
      g[i] = make_float4(gv[j].x / c - rv[j].x * k, gv[j].y / c - rv[j].y * k, gv[j].z / c - rv[j].z * k,
                         gv[j].w / c - rv[j].w * k);
  }
  for (int64_t i = lane + 64 * kRegs; i < D4; i += 64) {
    const uint2 w = r[i];
    const float4 gg = g[i];
    g[i] = make_float4(gg.x / c - lo_f32(w.x) * k, gg.y / c - hi_f32(w.x) * k, gg.z / c - lo_f32(w.y) * k,
                       gg.w / c - hi_f32(w.y) * k);
  }
}

// out[i] = bf16(sum_s part[s][i]) widened to fp32: the reference's gradient
// contractions are bf16 dots (their outputs bf16), split over K here
__global__ __launch_bounds__(256) void bwd_sum_kernel(const float* __restrict__ part, int S, int64_t n,
                                                      float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float a = 0.f;
  for (int s = 0; s < S; ++s) a += part[static_cast<int64_t>(s) * n + i];
  out[i] = round_bf16(a);
}

struct BGemm {
  int64_t M, Nc, K;  // out [M, Nc] = A [M, K] . B [Nc, K]^T
  int RT, DT, spc;
  int nbf;           // tile width 64 nbf (tiled_write_kernel<nbf>)
};

BGemm bgemm(int64_t M, int64_t Nc, int64_t K) {
  // output tiles 256 x 192 where that pads the Nc side less than 256 x 256
  // (Nc = 384: two tiles either way, a quarter of the wider ones' MFMAs idle)
  const int64_t p256 = (Nc + 255) / 256 * 256, p192 = (Nc + 191) / 192 * 192;
  const int nbf = p192 < p256 ? 3 : 4;
  BGemm g{M, Nc, K, static_cast<int>((M + kGRows - 1) / kGRows), static_cast<int>((Nc + 64 * nbf - 1) / (64 * nbf)),
          1, nbf};
  const int64_t blocks = (K + kGK - 1) / kGK, tiles = static_cast<int64_t>(g.RT) * g.DT;
  // K splits: the fewest that minimise the busiest CU's k blocks (rounds of
  // 256 workgroups x blocks per split) plus the fp32 partials' write and read
  // back, priced at ~1.6 us per k block and ~5 TB/s.  One split writes the
  // bf16-rounded result directly.  (Know-pool gradient GEMMs with K = T: 198
  // tiles, where two splits take as many block rounds as one.)
  double best = 0.0;
  int64_t spc = 1;
  for (int64_t c = 1; c <= 64 && c <= blocks; ++c) {
    const int64_t rounds = (tiles * c + 255) / 256, per = (blocks + c - 1) / c;
    const double cost = 1.6 * static_cast<double>(rounds * per) +
                        (c > 1 ? 2.0 * c * M * Nc * 4 / 5.0e6 : 0.0);  // us
    if (c == 1 || cost < best) {
      best = cost;
      spc = c;
    }
  }
  g.spc = static_cast<int>(spc);
  return g;
}

// Products that run as one launch (the backward's five gradient products):
// each product's K splits re-picked for the batch -- the fewest whose
// workgroups carry no more k blocks than the batch's mean per CU (the
// products' k blocks over 256 CUs, one workgroup per CU at a time).  With
// the longest workgroups dispatched first (tiled_backward orders the batch
// so), no CU's last workgroup then runs far past that mean, and fewer
// splits write and read back fewer fp32 partials.  (Know pool, T = 4096: d x
// and d h in two splits of 197 k blocks beside a mean of 247, where the
// per-product model took eight.)
void batch_splits(BGemm* const* gs, int n) {
  int64_t total = 0;
  for (int i = 0; i < n; ++i)
    total += static_cast<int64_t>(gs[i]->RT) * gs[i]->DT * ((gs[i]->K + kGK - 1) / kGK);
  const int64_t mean = (total + 255) / 256;
  for (int i = 0; i < n; ++i) {
    const int64_t blocks = (gs[i]->K + kGK - 1) / kGK;
    int64_t c = 1;
    while (c < 64 && c < blocks && (blocks + c - 1) / c > mean) ++c;
    gs[i]->spc = static_cast<int>(c);
  }
}

// bf16 src [rows, cols] -> dst [cols, rows_pad] (zero rows past `rows`), 64 x
// 64 tiles, 16-byte loads along src rows and 16-byte stores along dst rows
// (cols a multiple of 8)
__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ src,
                                                          uint16_t* __restrict__ dst, int64_t rows,
                                                          int64_t rows_pad, int64_t cols) {
  __shared__ uint16_t tile[64][72];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64, c0 = static_cast<int64_t>(blockIdx.y) * 64;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int idx = threadIdx.x + 256 * k;  // 512 pieces: 64 rows x 8
    const int r = idx >> 3, q = idx & 7;
    const int64_t row = r0 + r, col = c0 + 8 * q;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (row < rows && col < cols) v = *reinterpret_cast<const u32x4_t*>(src + row * cols + col);
    *reinterpret_cast<u32x4_t*>(&tile[r][8 * q]) = v;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int idx = threadIdx.x + 256 * k;  // 512 pieces: 64 dst rows x 8
    const int c = idx >> 3, q = idx & 7;
    const int64_t col = c0 + c, row = r0 + 8 * q;
    if (col >= cols || row >= rows_pad) continue;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = static_cast<uint32_t>(tile[8 * q + 2 * e][c]) | (static_cast<uint32_t>(tile[8 * q + 2 * e + 1][c]) << 16);
    *reinterpret_cast<u32x4_t*>(dst + col * rows_pad + row) = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

// src [rows, cols] -> dst [cols, rows_pad] (zero rows past `rows`)
hipError_t transpose(const uint16_t* src, uint16_t* dst, int64_t rows, int64_t rows_pad, int64_t cols,
                     hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(rows_pad / 64), static_cast<unsigned>((cols + 63) / 64));
  hipLaunchKernelGGL(transpose16_kernel, grid, dim3(256), 0, s, src, dst, rows, rows_pad, cols);
  return hipGetLastError();
}

// out [M, Nc] (fp32, bf16-rounded) = A [M, K] . B [Nc, K]^T, both with row
// stride ld (elements), zero past K: the write kernel's parameters (one
// split: the rounded result straight into out; else fp32 partials in part)
TWriteParams bwd_params(const BGemm& g, const uint16_t* A, const uint16_t* B, int64_t ld, float* part, float* out) {
  TWriteParams wp{};
  wp.P = A;
  wp.wt = B;
  wp.out_part = g.spc == 1 ? out : part;
  wp.Tv = g.M;
  wp.N = g.K;
  wp.N64 = ld;
  wp.D = g.Nc;
  wp.cs = g.K;
  wp.nc = 1;
  wp.spc = g.spc;
  wp.S = g.spc;
  wp.RT = g.RT;
  wp.DT = g.DT;
  wp.round_out = g.spc == 1;
  return wp;
}
unsigned bwd_grid(const BGemm& g) {
  return static_cast<unsigned>(8 * g.DT * ((static_cast<int64_t>(g.RT) * g.spc + 7) / 8));
}
hipError_t bwd_sum(const BGemm& g, const float* part, float* out, hipStream_t s) {
  if (g.spc == 1) return hipSuccess;
  const int64_t n = g.M * g.Nc;
  hipLaunchKernelGGL(bwd_sum_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, part, g.spc, n,
                     out);
  return hipGetLastError();
}

// The gradient contractions: one launch for all of them when their tiles
// have one width (the products' workgroups then fill the CUs that one
// product's last round leaves idle), else one launch each; split products'
// partials (part[i], disjoint) summed after.
hipError_t bwd_gemms(const BGemm* g, const uint16_t* const* A, const uint16_t* const* B, const int64_t* ld,
                     float* const* part, float* const* out, int n, hipStream_t s) {
  bool same = n <= kWriteBatch;
  for (int i = 1; i < n; ++i) same = same && g[i].nbf == g[0].nbf;
  if (same) {
    TWriteBatch b{};
    b.n = n;
    b.start[0] = 0;
    for (int i = 0; i < n; ++i) {
      b.p[i] = bwd_params(g[i], A[i], B[i], ld[i], part[i], out[i]);
      b.start[i + 1] = b.start[i] + static_cast<int>(bwd_grid(g[i]));
    }
    if (g[0].nbf == 3)
      hipLaunchKernelGGL(tiled_write_batch_kernel<3>, dim3(static_cast<unsigned>(b.start[n])), dim3(kGThreads),
                         gemm_lds(3), s, b);
    else
      hipLaunchKernelGGL(tiled_write_batch_kernel<4>, dim3(static_cast<unsigned>(b.start[n])), dim3(kGThreads),
                         kGemmLds, s, b);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  } else {
    for (int i = 0; i < n; ++i) {
      const TWriteParams wp = bwd_params(g[i], A[i], B[i], ld[i], part[i], out[i]);
      if (g[i].nbf == 3)
        hipLaunchKernelGGL((tiled_write_kernel<3, true>), dim3(bwd_grid(g[i])), dim3(kGThreads), gemm_lds(3), s, wp);
      else
        hipLaunchKernelGGL((tiled_write_kernel<4, true>), dim3(bwd_grid(g[i])), dim3(kGThreads), kGemmLds, s, wp);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  for (int i = 0; i < n; ++i) {
    hipError_t e = bwd_sum(g[i], part[i], out[i], s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

struct BLayout {
  size_t S, XR, DP, DXR, DS, PT, DXRT, DST, ET, RT, HT, XT, DRAWT, DRAW, RN, WN;
  size_t mom, inten_part, dm_part, dmz_part, tokv, psum, pmax, pn, dead, blk, coef, part, total;
  int64_t Tv, T64, Tv64, N64;
  int CT, RTv, RTt, NB, TS, nblk;
  int S_st;  // moment partials per row
  BGemm g_dw, g_dh, g_dx, g_de, g_dr;
};

BLayout blayout(const srw_desc_t& d) {
  BLayout l{};
  const int64_t T = d.T, N = d.n_units, D = d.d_model, dr = d.d_route, R = d.n_routes;
  l.Tv = T * R;
  l.T64 = (T + kNAlign - 1) / kNAlign * kNAlign;
  l.Tv64 = (l.Tv + kNAlign - 1) / kNAlign * kNAlign;
  l.N64 = (N + kNAlign - 1) / kNAlign * kNAlign;
  l.CT = static_cast<int>((N + kGRows - 1) / kGRows);
  l.RTv = static_cast<int>((l.Tv + kGRows - 1) / kGRows);
  l.RTt = static_cast<int>((T + kGRows - 1) / kGRows);
  l.NB = static_cast<int>(l.N64 / kTile);   // unit blocks of the elementwise passes
  l.TS = static_cast<int>(l.Tv64 / kTile);  // row blocks
  l.nblk = static_cast<int>((l.N64 + 255) / 256);
  l.g_dw = bgemm(N, D, l.Tv);
  l.g_dh = bgemm(l.Tv, dr, N);
  l.g_dx = bgemm(T, D, N);
  l.g_de = bgemm(N, dr, l.Tv);
  l.g_dr = bgemm(N, D, T);
  {
    // one launch when the five share a tile width (bwd_gemms)
    BGemm* const gs[5] = {&l.g_dw, &l.g_dr, &l.g_de, &l.g_dx, &l.g_dh};
    bool one = 5 <= kWriteBatch;
    for (int i = 1; i < 5; ++i) one = one && gs[i]->nbf == gs[0]->nbf;
    if (one) batch_splits(gs, 5);
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += al256(static_cast<int64_t>(bytes));
    return at;
  };
  const size_t vn = static_cast<size_t>(l.Tv) * l.N64 * 2, tn = static_cast<size_t>(T) * l.N64 * 2;
  l.S = take(vn);
  l.XR = take(tn);
  l.DP = take(vn);
  l.DXR = take(tn);
  l.DS = take(vn);
  l.PT = take(static_cast<size_t>(l.N64) * l.Tv64 * 2);
  l.DXRT = take(static_cast<size_t>(l.N64) * l.T64 * 2);
  l.DST = take(static_cast<size_t>(l.N64) * l.Tv64 * 2);
  l.ET = take(static_cast<size_t>(dr) * l.N64 * 2);
  l.RT = take(static_cast<size_t>(D) * l.N64 * 2);
  l.HT = take(static_cast<size_t>(dr) * l.Tv64 * 2);
  l.XT = take(static_cast<size_t>(D) * l.T64 * 2);
  l.DRAWT = take(static_cast<size_t>(D) * l.Tv64 * 2);
  l.DRAW = take(static_cast<size_t>(l.Tv) * D * 2);
  // the v4.0.1 gate: the forward-normalised read and write rows (v401:300-301)
  const bool gl = d.gate == SRW_GATE_GELU_V401;
  l.RN = take(gl ? static_cast<size_t>(N) * D * 2 : 0);
  l.WN = take(gl ? static_cast<size_t>(N) * D * 2 : 0);
  l.S_st = rows_gemm_supports(dr) ? rows_gemm_splits(l.Tv, N) : 2 * l.CT;
  l.mom = take(static_cast<size_t>(l.S_st) * l.Tv * 2 * 4);
  l.inten_part = take(static_cast<size_t>(l.NB) * l.Tv * 4);
  l.dm_part = take(static_cast<size_t>(l.NB) * l.Tv * 4);
  l.dmz_part = take(gl ? static_cast<size_t>(l.NB) * l.Tv * 4 : 0);
  l.tokv = take(static_cast<size_t>(l.Tv) * 9 * 4);
  l.psum = take(static_cast<size_t>(l.TS) * l.N64 * 4);
  l.pmax = take(static_cast<size_t>(l.TS) * l.N64 * 4);
  l.pn = take(static_cast<size_t>(l.N64) * 4);
  l.dead = take(static_cast<size_t>(l.N64) * 4);
  l.blk = take(static_cast<size_t>(l.nblk) * 2 * 4);
  l.coef = take(4 * 4);
  // one fp32 partial region per split product (they run in one launch)
  size_t part = 0;
  for (const BGemm& g : {l.g_dw, l.g_dr, l.g_de, l.g_dx, l.g_dh})
    if (g.spc > 1) part += al256(static_cast<int64_t>(g.spc) * g.M * g.Nc * 4);
  l.part = take(part);
  l.total = off;
  return l;
}

hipError_t store_gemm(const uint16_t* A, const uint16_t* B, uint16_t* C, int64_t rows, int64_t rows_b, int div,
                      int64_t N, int64_t N64, int64_t K, hipStream_t s) {
  TStoreParams p{};
  p.A = A;
  p.B = B;
  p.C = C;
  p.rows = rows;
  p.rows_b = rows_b;
  p.N = N;
  p.N64 = N64;
  p.K = K;
  p.div = div;
  p.RT = static_cast<int>((rows + kGRows - 1) / kGRows);
  p.CT = static_cast<int>((N + kGRows - 1) / kGRows);
  const unsigned grid = static_cast<unsigned>(8 * p.RT * ((p.CT + 7) / 8));
  hipLaunchKernelGGL(tiled_store_kernel, dim3(grid), dim3(kGThreads), kGemmLds, s, p);
  return hipGetLastError();
}

}  // namespace

bool tiled_backward_supports(const srw_desc_t& d) {
  if (d.dtype != SRW_BF16 || d.stats_mode != SRW_STATS_ONEPASS) return false;
  if (d.gate != SRW_GATE_V41 && d.gate != SRW_GATE_GELU_V401) return false;
  if (d.n_routes != 1 && d.n_routes != 2) return false;
  if (d.d_model % kNAlign != 0 || d.d_route % kNAlign != 0) return false;
  if (d.flags & (SRW_FLAG_EMULATE | SRW_FLAG_NO_FAST | SRW_FLAG_SPARSE_SKIP)) return false;
  if (!tile_offsets_fit(d.n_units) || !tile_offsets_fit(d.T * d.n_routes)) return false;
  return d.scale != 0.0f;
}

size_t tiled_backward_workspace_bytes(const srw_desc_t& d) { return blayout(d).total; }

hipError_t tiled_backward(const BackwardArgs& a) {
  const srw_desc_t& d = a.d;
  const BLayout l = blayout(d);
  const int R = d.n_routes;
  const int64_t T = d.T, N = d.n_units, D = d.d_model, dr = d.d_route, N64 = l.N64, Tv = l.Tv;
  auto b16 = [&](size_t off) { return reinterpret_cast<uint16_t*>(a.ws + off); };
  auto f32 = [&](size_t off) { return reinterpret_cast<float*>(a.ws + off); };
  uint16_t *S = b16(l.S), *XR = b16(l.XR), *DP = b16(l.DP), *DXR = b16(l.DXR), *DS = b16(l.DS);
  uint16_t *PT = b16(l.PT), *DXRT = b16(l.DXRT), *DST = b16(l.DST), *ET = b16(l.ET), *RT = b16(l.RT);
  uint16_t *HT = b16(l.HT), *XT = b16(l.XT), *DRAWT = b16(l.DRAWT), *DRAW = b16(l.DRAW);
  float *mom = f32(l.mom), *inten_part = f32(l.inten_part), *dm_part = f32(l.dm_part);
  float *tokv = f32(l.tokv), *psum = f32(l.psum), *pmax = f32(l.pmax), *pn = f32(l.pn), *dead = f32(l.dead);
  float *blk = f32(l.blk), *coef = f32(l.coef), *part = f32(l.part);
  float *mean = tokv, *var = tokv + Tv, *sdev = tokv + 2 * Tv, *tau = tokv + 3 * Tv, *dden = tokv + 4 * Tv;
  float *alpha = tokv + 5 * Tv, *beta = tokv + 6 * Tv, *zsum = tokv + 7 * Tv, *dsc = tokv + 8 * Tv;
  const auto* emb = static_cast<const uint16_t*>(a.in.emb);
  const bool gl = d.gate == SRW_GATE_GELU_V401;
  // the rows the products use: the v4.0.1 gate's forward-normalised ones
  const auto* read = static_cast<const uint16_t*>(a.in.read);
  const auto* write = static_cast<const uint16_t*>(a.in.write);
  const auto* x = static_cast<const uint16_t*>(a.in.x);
  const auto* h = static_cast<const uint16_t*>(a.in.h);
  const float exp_scale = -d.sharpness * 1.4426950408889634f;
  hipStream_t st = a.stream;
  hipError_t e;
  for (const void* fn : {reinterpret_cast<const void*>(tiled_stats_kernel),
                         reinterpret_cast<const void*>(tiled_store_kernel),
                         reinterpret_cast<const void*>(tiled_write_kernel<4>)})
    if ((e = set_lds(fn)) != hipSuccess) return e;
  if ((e = set_lds(reinterpret_cast<const void*>(tiled_write_kernel<3, true>), gemm_lds(3))) != hipSuccess) return e;
  if ((e = set_lds(reinterpret_cast<const void*>(tiled_write_kernel<4, true>))) != hipSuccess) return e;
  if ((e = set_lds(reinterpret_cast<const void*>(tiled_write_batch_kernel<3>), gemm_lds(3))) != hipSuccess) return e;
  if ((e = set_lds(reinterpret_cast<const void*>(tiled_write_batch_kernel<4>))) != hipSuccess) return e;
#define SRW_TRY(expr) \
  if ((e = (expr)) != hipSuccess) return e
  if (gl) {
    SRW_TRY(normalize_rows_bf16(static_cast<const uint16_t*>(a.in.read), b16(l.RN), N, D, st));
    SRW_TRY(normalize_rows_bf16(static_cast<const uint16_t*>(a.in.write), b16(l.WN), N, D, st));
    read = b16(l.RN);
    write = b16(l.WN);
  }
  // operands of the K = units / K = rows contractions, unit- or row-contiguous
  SRW_TRY(transpose(emb, ET, N, N64, dr, st));
  SRW_TRY(transpose(read, RT, N, N64, D, st));
  SRW_TRY(transpose(h, HT, Tv, l.Tv64, dr, st));
  SRW_TRY(transpose(x, XT, T, l.T64, D, st));

  // forward recompute: scores (stored), moments, tau, x.r (stored).  The
  // three [rows, N64] products with K = d_route or d_model (scores, x.r and
  // dP below) run on the moments kernel's tile loop where it takes that K
  // (rows_gemm: 128-row tiles, about two workgroups per CU), else on the
  // 256 x 256 tiles here.
  if (rows_gemm_supports(dr)) {
    SRW_TRY(rows_gemm(h, Tv, emb, N, dr, S, N64, mom, st));
  } else {
    TStatsParams sp{};
    sp.h = h;
    sp.emb = emb;
    sp.S = S;
    sp.mom = mom;
    sp.Tv = Tv;
    sp.N = N;
    sp.N64 = N64;
    sp.dr = dr;
    sp.RT = l.RTv;
    sp.CT = l.CT;
    hipLaunchKernelGGL(tiled_stats_kernel, dim3(static_cast<unsigned>(8 * l.RTv * ((l.CT + 7) / 8))),
                       dim3(kGThreads), kGemmLds, st, sp);
    SRW_TRY(hipGetLastError());
  }
  hipLaunchKernelGGL(bwd_token_stats_kernel, dim3(static_cast<unsigned>((Tv + 3) / 4)), dim3(256), 0, st, mom,
                     l.S_st, Tv, N, a.in.tau_offset, mean, var, sdev, tau);
  SRW_TRY(hipGetLastError());
  if (rows_gemm_supports(D)) {
    SRW_TRY(rows_gemm(x, T, read, N, D, XR, N64, nullptr, st));
  } else {
    SRW_TRY(store_gemm(read, x, XR, T, T, 1, N, N64, D, st));
  }

  // E1: gates, P^T, sum intensity, per-unit statistics
  ElemParams ep{};
  ep.S = S;
  ep.XR = XR;
  ep.DP = DP;
  ep.tau = tau;
  ep.dden = dden;
  ep.PT = PT;
  ep.inten_part = inten_part;
  ep.psum = psum;
  ep.pmax = pmax;
  ep.DXR = DXR;
  ep.DXRT = DXRT;
  ep.dm_part = dm_part;
  ep.dmz_part = gl ? f32(l.dmz_part) : nullptr;
  ep.sdev = sdev;
  ep.Tv = Tv;
  ep.N = N;
  ep.N64 = N64;
  ep.Tv64 = l.Tv64;
  ep.T64 = l.T64;
  ep.routes = R;
  ep.gp = a.gp;
  ep.exp_scale = exp_scale;
  ep.sharp = d.sharpness;
  const dim3 grid_e(static_cast<unsigned>(l.NB), static_cast<unsigned>(l.TS));
  // the forward's den and unit statistics given: no E1 pass (P^T comes from
  // the E2 pass's gates)
  const bool res = a.cot.den && a.cot.unit_diag;
  const float* zs = zsum;
  if (res) {
    zs = a.cot.den;  // den = max(sum intensity (v4.0.1: gate), 1): the den term's test sum > 1 reads the same on it
    hipLaunchKernelGGL(bwd_unit_from_diag_kernel, dim3(static_cast<unsigned>(l.nblk)), dim3(256), 0, st,
                       a.cot.unit_diag, Tv, N, N64, d.dead_threshold, pn, dead, blk);
    SRW_TRY(hipGetLastError());
  } else {
    if (gl) hipLaunchKernelGGL(bwd_fwd_elem_kernel<true>, grid_e, dim3(256), 0, st, ep);
    else hipLaunchKernelGGL(bwd_fwd_elem_kernel<false>, grid_e, dim3(256), 0, st, ep);
    SRW_TRY(hipGetLastError());
    hipLaunchKernelGGL(bwd_rowsum_kernel, dim3(static_cast<unsigned>((Tv + 63) / 64)), dim3(256), 0, st, inten_part,
                       l.NB, Tv, zsum);
    SRW_TRY(hipGetLastError());
    hipLaunchKernelGGL(bwd_unit_reduce_kernel, dim3(static_cast<unsigned>(l.nblk)), dim3(256), 0, st, psum, pmax,
                       l.TS, Tv, N, N64, d.dead_threshold, pn, dead, blk);
    SRW_TRY(hipGetLastError());
  }
  hipLaunchKernelGGL(bwd_unit_coef_kernel, dim3(1), dim3(256), 0, st, blk, l.nblk, N, a.cot.d_score_lb, coef);
  SRW_TRY(hipGetLastError());

  // cotangent of the chunk dots and the den term; dP; E2: the gate derivative
  hipLaunchKernelGGL(bwd_prep_kernel, dim3(static_cast<unsigned>(Tv)), dim3(256), 0, st, a.cot.d_out,
                     static_cast<const uint16_t*>(a.cot.out), zs, 1, d.scale, static_cast<int>(D), DRAW, dden,
                     dsc);
  SRW_TRY(hipGetLastError());
  if (a.g.dscale) {
    hipLaunchKernelGGL(bwd_total_kernel, dim3(1), dim3(256), 0, st, dsc, Tv, a.g.dscale);
    SRW_TRY(hipGetLastError());
  }
  dominant_kernel_begin(st);
  if (rows_gemm_supports(D)) {
    SRW_TRY(rows_gemm(DRAW, Tv, write, N, D, DP, N64, nullptr, st));
  } else {
    SRW_TRY(store_gemm(write, DRAW, DP, Tv, Tv, 1, N, N64, D, st));
  }
  dominant_kernel_end(st);
  if (res && gl)
    hipLaunchKernelGGL((bwd_gate_elem_kernel<true, true>), grid_e, dim3(256), 0, st, ep);
  else if (res)
    hipLaunchKernelGGL(bwd_gate_elem_kernel<true>, grid_e, dim3(256), 0, st, ep);
  else if (gl)
    hipLaunchKernelGGL((bwd_gate_elem_kernel<false, true>), grid_e, dim3(256), 0, st, ep);
  else
    hipLaunchKernelGGL(bwd_gate_elem_kernel<false>, grid_e, dim3(256), 0, st, ep);
  SRW_TRY(hipGetLastError());
  hipLaunchKernelGGL(bwd_token_kernel, dim3(static_cast<unsigned>((Tv + kTokRows - 1) / kTokRows)), dim3(256), 0, st,
                     dm_part, ep.dmz_part, l.NB, Tv, N, a.in.tau_offset, mean, var, sdev, a.g.dtau_offset, alpha,
                     beta);
  SRW_TRY(hipGetLastError());
  // E3: ds in both layouts
  DsParams dp{};
  dp.S = S;
  dp.XR = XR;
  dp.DP = DP;
  dp.tau = tau;
  dp.dden = dden;
  dp.alpha = alpha;
  dp.beta = beta;
  dp.pn = pn;
  dp.dead = dead;
  dp.coef = coef;
  dp.DS = DS;
  dp.DST = DST;
  dp.sdev = sdev;
  dp.d_pen = a.cot.d_dead_penalty;
  dp.Tv = Tv;
  dp.N = N;
  dp.N64 = N64;
  dp.Tv64 = l.Tv64;
  dp.routes = R;
  dp.gp = a.gp;
  dp.exp_scale = exp_scale;
  dp.sharp = d.sharpness;
  if (gl) hipLaunchKernelGGL(bwd_ds_elem_kernel<true>, grid_e, dim3(256), 0, st, dp);
  else hipLaunchKernelGGL(bwd_ds_elem_kernel<false>, grid_e, dim3(256), 0, st, dp);
  SRW_TRY(hipGetLastError());

  // the five gradient contractions: bf16 dots, fp32 accumulation
  SRW_TRY(transpose(DRAW, DRAWT, Tv, l.Tv64, D, st));
  {
    BGemm gs[5] = {l.g_dw, l.g_dr, l.g_de, l.g_dx, l.g_dh};
    const uint16_t* As[5] = {PT, DXRT, DST, DXR, DS};
    const uint16_t* Bs[5] = {DRAWT, XT, HT, RT, ET};
    int64_t lds_[5] = {l.Tv64, l.T64, l.Tv64, N64, N64};
    float* outs[5] = {a.g.dwrite, a.g.dread, a.g.demb, a.g.dx, a.g.dh};
    // the products with the longest workgroups (k blocks per split) first
    // (stable insertion sort of the five)
    auto wg_blocks = [](const BGemm& g) { return ((g.K + kGK - 1) / kGK + g.spc - 1) / g.spc; };
    for (int i = 1; i < 5; ++i)
      for (int j = i; j > 0 && wg_blocks(gs[j]) > wg_blocks(gs[j - 1]); --j) {
        std::swap(gs[j], gs[j - 1]);
        std::swap(As[j], As[j - 1]);
        std::swap(Bs[j], Bs[j - 1]);
        std::swap(lds_[j], lds_[j - 1]);
        std::swap(outs[j], outs[j - 1]);
      }
    float* parts[5];
    float* pp = part;
    for (int i = 0; i < 5; ++i) {
      parts[i] = pp;
      if (gs[i].spc > 1) pp += al256(static_cast<int64_t>(gs[i].spc) * gs[i].M * gs[i].Nc * 4) / 4;
    }
    SRW_TRY(bwd_gemms(gs, As, Bs, lds_, parts, outs, 5, st));
  }
  if (gl) {  // d read / d write through the forward normalisation
    const dim3 grid_n(static_cast<unsigned>((N + 3) / 4));
    hipLaunchKernelGGL(bwd_norm_rows_kernel, grid_n, dim3(256), 0, st, static_cast<const uint16_t*>(a.in.read),
                       a.g.dread, N, D);
    SRW_TRY(hipGetLastError());
    hipLaunchKernelGGL(bwd_norm_rows_kernel, grid_n, dim3(256), 0, st, static_cast<const uint16_t*>(a.in.write),
                       a.g.dwrite, N, D);
    SRW_TRY(hipGetLastError());
  }
#undef SRW_TRY
  return hipSuccess;
}

}  // namespace srw

// bf16/fp16 GEMM on CDNA4 matrix cores, plus a strided SIMT fallback.
//
// gemm_nt:  C[M,N] = alpha * A[M,K] . B[N,K]^T (+ C if accumulate), both operands K-contiguous
// (the layout of X and of a row-major weight W[N,K] in Y = X W^T); fp32 accumulation, output in
// bf16/fp16/fp32.
//
// Main path (K % 64 == 0), gemm_nt_v4_kernel: v_mfma_f32_16x16x32 (on MI355X it sustains a higher
// rate than the 32x32x16 form under the board power limit with random data), 8 waves per
// 256 x 256 x 64 tile (each 64 x 128) or 4 waves for 128 x 128 tiles, picked so the grid
// still covers the 256 CUs.  Operand tiles go global -> LDS with wave-wide global_load_lds_dwordx4
// into a ring of k-tiles (no register staging); LDS rows are unpadded and XOR-swizzled so the
// fragment reads are bank-conflict free; fragment reads are software-pipelined one k-step ahead.
// Workgroup ids are remapped so that each XCD (ids congruent mod 8) owns a contiguous range of
// output tiles, rastered in groups of 8 tile-rows so concurrently running tiles share operand rows
// in that XCD's L2.
//
// K % 64 != 0: gemm_nt_kernel, a register-staged 256 x 128 x 64 tile with padded LDS rows and
// v_mfma_f32_32x32x16 (the k tail is zero-filled).
#include <type_traits>

#include "common.h"

namespace {

constexpr int kThreads = 256;

template <typename T> Q3_DEV f32x16 mfma_32x32x16(bf16x8_t a, bf16x8_t b, f32x16 c);
template <> Q3_DEV f32x16 mfma_32x32x16<BF16>(bf16x8_t a, bf16x8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <> Q3_DEV f32x16 mfma_32x32x16<F16>(bf16x8_t a, bf16x8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                 0, 0, 0);
}

// Maps a linear workgroup id to (tile_m, tile_n): XCD-contiguous ranges, then GROUP-row raster.
Q3_DEV void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GROUP = 4;  // measured on the layer-step shapes: 4 < 6 < 8 < 2 < 16 < 1 (total time)
  const int total = tiles_m * tiles_n;
  if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  const int width = GROUP * tiles_n;
  const int first = (bid / width) * GROUP;
  const int gsize = min(tiles_m - first, GROUP);
  tm = first + (bid % width) % gsize;
  tn = (bid % width) / gsize;
}

template <typename T, typename O, int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(const u16* __restrict__ A, const u16* __restrict__ B,
                                                           typename O::storage* __restrict__ C, int M, int N, int K,
                                                           int64_t lda, int64_t ldb, int64_t ldc, float alpha,
                                                           int accumulate) {
  constexpr int LDK = BK + 8;
  constexpr int WAVES_N = BN / WN;
  static_assert((BM / WM) * WAVES_N == 4, "4 waves per workgroup");
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int CPR = BK / 8;                   // 16-byte chunks per tile row
  constexpr int RSTEP = kThreads / CPR;         // tile rows covered per load step
  constexpr int A_LOADS = BM / RSTEP, B_LOADS = BN / RSTEP;
  __shared__ __attribute__((aligned(16))) u16 lds[2][(BM + BN) * LDK];

  int tm, tn;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int ck = tid % CPR, cr = tid / CPR;

  i32x4 ra[A_LOADS], rb[B_LOADS];
  auto gload = [&](int k0) {
    const int kk = k0 + ck * 8;
    const bool kin = kk < K;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int row = m0 + cr + i * RSTEP;
      ra[i] = (kin && row < M) ? *reinterpret_cast<const i32x4*>(A + (int64_t)row * lda + kk) : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int row = n0 + cr + i * RSTEP;
      rb[i] = (kin && row < N) ? *reinterpret_cast<const i32x4*>(B + (int64_t)row * ldb + kk) : i32x4{0, 0, 0, 0};
    }
  };
  auto swrite = [&](int buf) {
    u16* la = lds[buf];
    u16* lb = la + BM * LDK;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) *reinterpret_cast<i32x4*>(la + (cr + i * RSTEP) * LDK + ck * 8) = ra[i];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) *reinterpret_cast<i32x4*>(lb + (cr + i * RSTEP) * LDK + ck * 8) = rb[i];
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = (K + BK - 1) / BK;
  gload(0);
  swrite(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
    const u16* la = lds[cur] + (wm * WM + (lane & 31)) * LDK + (lane >> 5) * 8;
    const u16* lb = lds[cur] + BM * LDK + (wn * WN + (lane & 31)) * LDK + (lane >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_t af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const bf16x8_t*>(la + i * 32 * LDK + ks * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = *reinterpret_cast<const bf16x8_t*>(lb + j * 32 * LDK + ks * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x16<T>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < nk) swrite(cur ^ 1);
    __syncthreads();
  }

  // Accumulator layout of a 32x32 MFMA tile: lane l, element v -> row 8*(v/4) + 4*(l/32) + v%4,
  // column l%32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * WN + j * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M && col < N) {
          typename O::storage* c = C + (int64_t)row * ldc + col;
          float r = alpha * acc[i][j][v];
          if (accumulate) r += to_f32<O>(*c);
          *c = from_f32<O>(r);
        }
      }
    }
}

// ---------------------------------------------------------------- direct-to-LDS ring helpers
// Workgroup barrier for a direct-to-LDS ring: this wave's loads older than its newest N have
// landed in LDS and its own LDS reads are done (vmcnt(N) lgkmcnt(0)), then s_barrier.
// __syncthreads() would add a release fence, which waits for vmcnt(0) and so drains every
// prefetched stage of the ring at each k-tile.
template <int N> Q3_DEV void ring_sync() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0 << 8));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- v4: register-lean 16x16x32 pipeline
// 128-byte LDS rows (BK = 64) with the 16-byte chunk swizzle swz(r) = r & 7.  A 16x16x32 fragment
// read has lanes 16q..16q+15 on 16 consecutive rows at one logical chunk; measured on MI355X this
// swizzle reads such fragments conflict free (~139 TB/s of LDS reads per chip in a read-only loop),
// while (r & 7) ^ ((r >> 3) & 1) or (r ^ (r >> 3)) & 7 conflict two ways (~76 TB/s).  Because every
// fragment starts on a multiple of 8 rows, all fragments of a wave share one swizzle: a fragment
// address is one per-k-step base register plus an immediate offset, which leaves room for a fenced
// double buffer of fragments (reads of k-step ks+1 in flight during the MFMAs of ks, the first
// reads of tile kt+1 during the last MFMAs of tile kt) at two waves per SIMD.
Q3_DEV int swz8(int r) { return r & 7; }
// 64-byte rows (BK = 32, 4 chunks): (r >> 1) & 3 is the conflict-free choice for the same read
// pattern (~133 TB/s; r & 3, (r >> 2) & 3 and the XOR mixes of them ~75 TB/s).
Q3_DEV int swz4(int r) { return (r >> 1) & 3; }
template <int CPR> Q3_DEV int gemm_swz(int r) {
  if constexpr (CPR == 8) return swz8(r);
  else return swz4(r);
}

// Cross-entropy gradient epilogue (EPI = 1): the tile is a chunk of logits z[m, col0 + n] and the
// kernel stores dz = (exp(z - lse[m]) - [col0 + n == tgt[m]]) * (*up) / (*count) instead, 0 for rows
// whose target is ignore_index or outside [0, vocab) (the fp32 logits never reach memory).
// Statistics epilogue (EPI = 2, 128 columns per wave): per row and 128-column group p (= part0 +
// global column group of the tile), m_part[p * ldp + row] / s_part[...] get the group's max and
// sum of exp(z - max), and pick[row] the logit of column tgt[row] - col0 when it lies in this chunk.
// Gate/up epilogue (EPI = 3): the B operand is two weights, Wg (B) and Wu (b2), interleaved in
// 16-row blocks (virtual B row r: block r / 16, even blocks from Wg, odd from Wu, weight row
// (block / 2) * 16 + r % 16), so each lane holds the gate and up accumulators of the same output
// element in neighbouring 16 x 16 fragments.  It stores G = bf16(x Wg^T), U = bf16(x Wu^T) and
// Y = silu(G) * U computed from the rounded G and U (row stride ldc, C = Y).
// Segmented operand (EPI = 4): the B rows are the concatenation of up to 3 weights (the Q, K and V
// projections of one input) and each output column segment goes to its own matrix; every segment
// boundary is a multiple of BN, so a tile reads one weight and writes one output (plain EPI 0
// epilogue with that segment's pointers).
// SwiGLU-backward epilogue (EPI 5): the tile is dY = A B^T, the gradient of the SwiGLU output
// y = silu(g) * u (dOut W_down with B = W_down^T); it is rounded to the storage type as a standalone
// GEMM output would be, and the kernel stores dg = dY u s (1 + g (1 - s)) and du = dY g s (s = sigmoid(g),
// the formula of the SwiGLU backward kernel, so results are bit-identical to GEMM + that kernel),
// plus, when dgt is set, the transposes of dg and du -- the operands the weight-gradient GEMM needs.
struct CeEpi {
  const int64_t* tgt;
  const float* lse;
  const float* count;
  const float* up;
  int64_t col0, vocab, ignore;
  float* m_part;
  float* s_part;
  float* pick;
  int64_t part0, ldp;
  const u16* b2;
  u16* g_out;
  u16* u_out;
  u16* zt;       // EPI 1: optional transposed copy of dz ([N][M] at row stride ldzt)
  int64_t ldzt;
  // EPI 4: up to 3 column segments [seg_n0[s], seg_n0[s + 1]) of B / C, each its own weight and output
  const u16* seg_b[3];
  u16* seg_c[3];
  int64_t seg_ldc[3];
  int64_t seg_n0[3];
  int nseg;
  // EPI 5: SwiGLU inputs g / u [M, N] (row stride ldgu), gradients dg / du [M, N] (row stride lddgu) and
  // optionally their transposes dgt / dut [N, M] (row stride lddt)
  const u16* gin;
  const u16* uin;
  int64_t ldgu;
  u16* dgo;
  u16* duo;
  int64_t lddgu;
  u16* dgt;
  u16* dut;
  int64_t lddt;
  // EPI 0 (16-bit output, full 256 x 256 tiles): when set, C = res + the GEMM output (row stride ldres)
  const u16* res;
  int64_t ldres;
  // EPI 0 over a grid of gridDim.y K splits: split y multiplies the y-th K / gridDim.y slice and stores
  // its partial product at C + y * split_ld
  int64_t split_ld;
  // EPI 3: when set, also Y^T [N, M] (row stride ldyt), the down projection's weight-gradient operand
  u16* yt;
  int64_t ldyt;
  // EPI 2: when set, the logits rounded to the storage type are stored too (row stride ldzs), and the
  // statistics are formed from those rounded values
  u16* zs;
  int64_t ldzs;
};

Q3_DEV void lse_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * __expf(m - mn) + s2 * __expf(m2 - mn);
  m = mn;
}

template <typename T, typename O, int BM, int BN, int WM, int WN, int BK, int STAGES, bool EVEN, int EPI = 0>
__global__ __launch_bounds__(WM * WN * 64) void gemm_nt_v4_kernel(const u16* __restrict__ A,
                                                                  const u16* __restrict__ B,
                                                                  typename O::storage* __restrict__ C, int M, int N,
                                                                  int K, int64_t lda, int64_t ldb, int64_t ldc,
                                                                  float alpha, int accumulate, int vec_store,
                                                                  CeEpi ce) {
  static_assert(BK == 64 || BK == 32, "k tile");
  constexpr int NW = WM * WN, ROWB = BK * 2, CPR = BK / 8, RPL = 64 / CPR;
  constexpr int TMW = BM / WM, TNW = BN / WN, FM = TMW / 16, FN = TNW / 16;
  constexpr int RG = (BM + BN) / RPL;
  static_assert(RG % NW == 0 && (BM / RPL) % NW == 0, "row groups must split evenly over the waves");
  constexpr int LPW = RG / NW, A_LOADS = (BM / RPL) / NW;
  constexpr int STAGE = (BM + BN) * BK;  // elements
  constexpr int KS = BK / 32;            // k-steps of 32 per tile
  __shared__ __attribute__((aligned(1024))) u16 lds[STAGES * STAGE];

  int tm, tn;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  if constexpr (EPI == 0) {
    if (gridDim.y > 1) {  // K split: this workgroup's slice of K and its own partial output
      K /= (int)gridDim.y;
      A += (int64_t)blockIdx.y * K;
      B += (int64_t)blockIdx.y * K;
      C += (int64_t)blockIdx.y * ce.split_ld;
    }
  }
  if constexpr (EPI == 4) {  // this tile's weight and output, shifted so column n0 addresses them
    int sg = 0;
    while (sg + 1 < ce.nseg && n0 >= ce.seg_n0[sg + 1]) ++sg;
    B = ce.seg_b[sg] - ce.seg_n0[sg] * ldb;
    C = reinterpret_cast<typename O::storage*>(ce.seg_c[sg]) - ce.seg_n0[sg];
    ldc = ce.seg_ldc[sg];
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);

  // ---- global -> LDS: row R of the [A; B] stage, logical chunk c lands at physical c ^ swz8(R).
  // Row groups of 8 rows, so the swizzle (hence the lane offset) is the same for every group.
  const int csrc = (lane % CPR) ^ gemm_swz<CPR>(lane / CPR);  // logical chunk this lane fetches (row = lane / CPR)
  const uint32_t offa = (uint32_t)(((lane / CPR) * lda + csrc * 8) * 2);
  const uint32_t offb = (uint32_t)(((lane / CPR) * ldb + csrc * 8) * 2);
  const u16* src[EVEN ? 1 : LPW];
  if constexpr (!EVEN) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int R = (wave + NW * i) * RPL + lane / CPR;
      if (R < BM) src[i] = A + (int64_t)min(m0 + R, M - 1) * lda + csrc * 8;
      else src[i] = B + (int64_t)min(n0 + R - BM, N - 1) * ldb + csrc * 8;
    }
  }
  // Full tiles (EVEN): the ring refill is issued on every tile, so the loop body is straight-line
  // code and the refill loads interleave with the MFMAs; past the last k tile it re-reads a tile that
  // was just consumed (L2-resident) into a stage that is never read again.
  int kfill = 0;  // k of a tile already loaded: the data a refill past the last k tile re-reads
  auto issue = [&](int stage, int k0) {  // k0 < 0: past the last k tile (EVEN only)
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int rg = wave_u + NW * i;
      u16* dst = lds + stage * STAGE + rg * RPL * BK;
      if constexpr (EVEN) {
        const int kk = k0 < 0 ? kfill : k0;  // past the last k tile: refill with a resident tile's data
        const void* g;
        if (i < A_LOADS) {
          g = reinterpret_cast<const char*>(A + (int64_t)(m0 + rg * RPL) * lda + kk) + offa;
        } else if constexpr (EPI == 3) {
          const int vr = rg * RPL - BM, blk = vr >> 4;  // virtual B row within the tile
          const u16* w = (blk & 1) ? ce.b2 : B;
          g = reinterpret_cast<const char*>(w + (int64_t)(n0 / 2 + (blk >> 1) * 16 + (vr & 15)) * ldb + kk) + offb;
        } else {
          g = reinterpret_cast<const char*>(B + (int64_t)(n0 + rg * RPL - BM) * ldb + kk) + offb;
        }
        __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
      } else {
        const void* g = src[i] + k0;
        __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
      }
    }
  };

  // ---- LDS -> fragments.  Lane l reads row (fragment base + l % 16), logical chunk ks*4 + l/16.
  const int quarter = lane >> 4, sw = gemm_swz<CPR>(lane & 15);
  uint32_t va[KS], vb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const uint32_t coff = (uint32_t)(((ks * 4 + quarter) ^ sw) << 4);
    va[ks] = (uint32_t)((wm * TMW + (lane & 15)) * ROWB) + coff;
    vb[ks] = (uint32_t)((BM + wn * TNW + (lane & 15)) * ROWB) + coff;
  }
  const char* lds_c = reinterpret_cast<const char*>(lds);
  bf16x8_t af[2][FM], bfr[2][FN];
  auto load = [&](int stage, int buf, int ks) {
    const char* sb = lds_c + stage * (STAGE * 2);
#pragma unroll
    for (int i = 0; i < FM; ++i) af[buf][i] = *reinterpret_cast<const bf16x8_t*>(sb + va[ks] + i * 16 * ROWB);
#pragma unroll
    for (int j = 0; j < FN; ++j) bfr[buf][j] = *reinterpret_cast<const bf16x8_t*>(sb + vb[ks] + j * 16 * ROWB);
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = K / BK;
  if constexpr (EVEN) {  // every ring slot is always issued (past the end: zero-filling range misses)
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st) issue(st, st < nk ? st * BK : -1);
    ring_sync<(STAGES - 2) * LPW>();
    issue(STAGES - 1, STAGES - 1 < nk ? (STAGES - 1) * BK : -1);
  } else {
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st)
      if (st < nk) issue(st, st * BK);
    if (nk - 1 >= STAGES - 2) ring_sync<(STAGES - 2) * LPW>();
    else ring_sync<0>();
    if (STAGES - 1 < nk) issue(STAGES - 1, (STAGES - 1) * BK);
  }
  load(0, 0, 0);
  // One tile: each k-step first reads the next step's fragments into the other buffer (the next
  // tile's first step after the barrier that makes that tile resident and frees this tile's stage
  // for the ring refill), then runs its MFMAs.  CUR is the buffer holding step 0's fragments: with
  // an odd number of steps per tile it alternates, so tiles go in pairs to keep it a constant.
  auto tile = [&](int kt, auto cur_c) {
    constexpr int CUR = decltype(cur_c)::value;
    const int stage = kt % STAGES;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int b = (CUR + ks) & 1;
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 1 < KS) {
        // Step ks's fragments landed long ago: waiting for them keeps the outstanding-read count
        // within what the LDS counter tracks, so the MFMAs below need no wait.
        __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
        load(stage, b ^ 1, ks + 1);
      } else {
        // Tile kt+1 resident; every wave done with tile kt.  Runs on the last tile too (re-reading a
        // resident stage) so the LDS counter state is the same on every path into the MFMAs.
        if constexpr (EVEN) {
          ring_sync<(STAGES - 2) * LPW>();
          kfill = kt * BK;
          issue(stage, kt + STAGES < nk ? (kt + STAGES) * BK : -1);
        } else {
          if (kt + STAGES - 1 < nk) ring_sync<(STAGES - 2) * LPW>();
          else ring_sync<0>();
          if (kt + STAGES < nk) issue(stage, (kt + STAGES) * BK);
        }
        load((kt + 1) % STAGES, b ^ 1, 0);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma_16x16x32<T>(bfr[b][j], af[b][i], acc[i][j]);
      // Spread the step's memory instructions through its MFMAs.  Refill step: one ring refill load
      // per two MFMAs, then one fragment read (of the next tile's first step) per MFMA.  Other steps:
      // the next step's fragment reads start after 3/8 of the MFMAs, one per MFMA.  Measured on the
      // ten layer-step GEMM shapes against one load / one read per MFMA from the start of each step
      // (both steps alike): 6.45-6.48 against 6.58-6.59 ms in total; issuing all of them in one burst
      // after the barrier: 6.65 ms.
      if (ks + 1 == KS) {
#pragma unroll
        for (int q = 0; q < LPW; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
        }
#pragma unroll
        for (int q = 0; q < FM + FN; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        }
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN * 3 / 8, 0);
#pragma unroll
        for (int q = 0; q < FM + FN; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if constexpr (KS % 2 == 0) {
    for (int kt = 0; kt < nk; ++kt) tile(kt, std::integral_constant<int, 0>{});
  } else {
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
      tile(kt, std::integral_constant<int, 0>{});
      tile(kt + 1, std::integral_constant<int, 1>{});
    }
    if (kt < nk) tile(kt, std::integral_constant<int, 0>{});
  }

  // ---- epilogue: lane owns row m and 4 consecutive columns of each 16x16 block (C^T layout)
  // Coalesced epilogue through LDS (16-bit outputs of full tiles): each wave rounds its tile into a
  // private LDS block (16-byte chunks XOR-swizzled by row, conflict-free writes and reads), then
  // stores whole rows with 16-byte stores instead of 8-byte pieces of 16 rows.
  typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
  [[maybe_unused]] char* wl = reinterpret_cast<char*>(lds) + wave_u * (TMW * TNW * 2);
  // NC = columns of the staged tile (TNW, or TNW / 2 for one gate/up output)
  [[maybe_unused]] auto stage = [&](auto nc_c, int i, int jc, uint32_t lo, uint32_t hi) {
    constexpr int NC = decltype(nc_c)::value, CH = NC / 8;
    static_assert(CH == 8 || CH == 16, "the staging swizzle needs 8 or 16 16-byte chunks per row");
    const int r = i * 16 + (lane & 15);
    const int c = (jc * 16 + 4 * quarter) >> 3;  // logical 16-byte chunk
    const int sw = CH == 16 ? (r & 15) : ((r >> 1) & 7);
    *reinterpret_cast<i32x2*>(wl + r * (NC * 2) + ((c ^ sw) << 4) + (quarter & 1) * 8) = i32x2{(int)lo, (int)hi};
  };
  [[maybe_unused]] auto flush = [&](auto nc_c, typename O::storage* dst, int64_t ld, auto nr_c) {
    constexpr int NC = decltype(nc_c)::value, CH = NC / 8, RPI = 64 / CH;  // rows per instruction
    static_assert(CH == 8 || CH == 16, "the staging swizzle needs 8 or 16 16-byte chunks per row");
    constexpr int NR = decltype(nr_c)::value;
    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // this wave's staging writes
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int q = 0; q < NR / RPI; ++q) {
      const int r = q * RPI + lane / CH, c = lane % CH;
      const int sw = CH == 16 ? (r & 15) : ((r >> 1) & 7);
      const i32x4 v = *reinterpret_cast<const i32x4*>(wl + r * (NC * 2) + ((c ^ sw) << 4));
      *reinterpret_cast<i32x4*>(dst + (int64_t)r * ld + c * 8) = v;
    }
    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // reads done before the block is reused
    __builtin_amdgcn_wave_barrier();
  };
  if constexpr (EPI == 3) {
    static_assert(FN % 2 == 0 && EVEN, "gate/up fragments come in (gate, up) pairs of full tiles");
    static_assert(O::vec == 8, "16-bit outputs");
    constexpr auto NC = std::integral_constant<int, TNW / 2>{};
    __syncthreads();  // every wave is done with the operand ring
    const int64_t o0 = (int64_t)(m0 + wm * TMW) * ldc + (n0 + wn * TNW) / 2;
#pragma unroll
    for (int out = ce.g_out ? 0 : 2; out < 3; ++out) {  // G and U only when stored (training)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int p = 0; p < FN / 2; ++p) {
          float gq[4], uq[4], v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            gq[e] = to_f32<T>(from_f32<T>(acc[i][2 * p][e]));
            uq[e] = to_f32<T>(from_f32<T>(acc[i][2 * p + 1][e]));
            v[e] = out == 0 ? gq[e] : out == 1 ? uq[e] : gq[e] * q3_sigmoid(gq[e]) * uq[e];
          }
          stage(NC, i, p, pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]));
        }
      flush(NC, (out == 0 ? ce.g_out : out == 1 ? ce.u_out : C) + o0, ldc, std::integral_constant<int, TMW>{});
    }
    if (ce.yt) {
      // Y^T from the Y block still staged in the wave's LDS ([TMW rows][NC columns], 16-byte chunks
      // XOR-swizzled by row pair): the gfx950 transpose read gives lane j of a 16-lane group column
      // t0 + j of 4 consecutive rows (lanes address row R0 + a / 4, columns t0 + 4 (a % 4)); two reads
      // make 8 rows = one 16-byte store of a Y^T row.  Four groups take consecutive 8-row blocks.
      typedef short v4s_t __attribute__((ext_vector_type(4)));
      constexpr int NCV = decltype(NC)::value;
      const int j = lane & 15, grp = lane >> 4;
      const int64_t yrow0 = m0 + wm * TMW, ycol0 = (n0 + wn * TNW) / 2;
#pragma unroll
      for (int pi = 0; pi < (NCV / 16) * (TMW / 32); ++pi) {
        const int t0 = 16 * (pi % (NCV / 16)), r0 = 32 * (pi / (NCV / 16)) + 8 * grp;
        i32x4 v;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int row = r0 + 4 * hh + (j >> 2);
          const int cb = 2 * t0 + 8 * (j & 3);  // byte offset of the 4 columns in the row
          const char* pa = wl + row * (NCV * 2) + ((((cb >> 4) ^ ((row >> 1) & 7))) << 4) + (cb & 15);
          const i32x2 t = __builtin_bit_cast(
              i32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)pa));
          v[2 * hh] = t[0];
          v[2 * hh + 1] = t[1];
        }
        *reinterpret_cast<i32x4*>(ce.yt + (ycol0 + t0 + j) * ce.ldyt + yrow0 + r0) = v;
      }
    }
    return;
  }
  if constexpr (EPI == 5) {
    static_assert(EVEN && O::vec == 8 && TMW == 64 && TNW == 128, "full 256 x 256 tiles, 64 x 128 per wave");
    constexpr int CH = TNW / 8, RPI = 64 / CH, NQ = TMW / RPI;  // 16 chunks per row, 4 rows per pass, 16 passes
    __syncthreads();  // every wave is done with the operand ring
    // dY rounded to the storage type, staged row-major in the wave's block
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        stage(std::integral_constant<int, TNW>{}, i, j, pack2<O>(acc[i][j][0], acc[i][j][1]),
              pack2<O>(acc[i][j][2], acc[i][j][3]));
    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
    __builtin_amdgcn_wave_barrier();
    const int64_t row0 = m0 + wm * TMW, col0 = n0 + wn * TNW;
    const int c = lane % CH;
    i32x4 dgp[NQ], dup[NQ];
    // two halves of the rows: g / u loads of a half all in flight before the first use
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      i32x4 gv[NQ / 2], uv[NQ / 2], dv[NQ / 2];
#pragma unroll
      for (int q = 0; q < NQ / 2; ++q) {
        const int r = (hh * (NQ / 2) + q) * RPI + lane / CH;
        gv[q] = *reinterpret_cast<const i32x4*>(ce.gin + (row0 + r) * ce.ldgu + col0 + c * 8);
        uv[q] = *reinterpret_cast<const i32x4*>(ce.uin + (row0 + r) * ce.ldgu + col0 + c * 8);
        dv[q] = *reinterpret_cast<const i32x4*>(wl + r * (TNW * 2) + ((c ^ (r & 15)) << 4));
      }
#pragma unroll
      for (int q = 0; q < NQ / 2; ++q) {
        const int r = (hh * (NQ / 2) + q) * RPI + lane / CH;
        const Vec<O> gf = unpack_vec<O>(gv[q]), uf = unpack_vec<O>(uv[q]), df = unpack_vec<O>(dv[q]);
        Vec<O> og, ou;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float sg = q3_sigmoid(gf.v[e]);
          og.v[e] = df.v[e] * uf.v[e] * sg * (1.f + gf.v[e] * (1.f - sg));
          ou.v[e] = df.v[e] * gf.v[e] * sg;
        }
        i32x4 pg, pu;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          pg[w] = (int)pack2<O>(og.v[2 * w], og.v[2 * w + 1]);
          pu[w] = (int)pack2<O>(ou.v[2 * w], ou.v[2 * w + 1]);
        }
        *reinterpret_cast<i32x4*>(ce.dgo + (row0 + r) * ce.lddgu + col0 + c * 8) = pg;
        *reinterpret_cast<i32x4*>(ce.duo + (row0 + r) * ce.lddgu + col0 + c * 8) = pu;
        dgp[hh * (NQ / 2) + q] = pg;
        dup[hh * (NQ / 2) + q] = pu;
      }
    }
    if (ce.dgt) {
      // Transposed copies through the wave's block: the [64 rows][128 columns] gradient tile is written
      // row-major (16-byte stores, chunks XOR-swizzled by row), then read back transposed with the gfx950
      // LDS transpose read: in each 16-lane group, lane a addresses 4 columns of row R0 + a / 4, so lane j
      // receives column T0 + j of rows R0 .. R0 + 3 (a second read gives R0 + 4 .. R0 + 7), i.e. 16 bytes
      // of one row of the transposed output.  Four groups take consecutive 8-row blocks of one column
      // block, so every column's 64 transposed bytes are written by four lanes of one store.
      auto tstore = [&](const i32x4 (&p)[NQ], u16* dst) {
        __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // earlier reads of the block done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const int r = q * RPI + lane / CH;
          *reinterpret_cast<i32x4*>(wl + r * (TNW * 2) + ((c ^ (r & 15)) << 4)) = p[q];
        }
        __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
        __builtin_amdgcn_wave_barrier();
        const int j = lane & 15, grp = lane >> 4;
#pragma unroll
        for (int pi = 0; pi < (TNW / 16) * (TMW / 32); ++pi) {
          const int t0 = 16 * (pi % (TNW / 16)), r0 = 32 * (pi / (TNW / 16)) + 8 * grp;
          i32x4 v;
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const int row = r0 + 4 * hh + (j >> 2);
            const int cb = 2 * t0 + 8 * (j & 3);  // byte offset of the 4 columns in the row
            const char* pa = wl + row * (TNW * 2) + ((((cb >> 4) ^ (row & 15))) << 4) + (cb & 15);
            typedef short v4s_t __attribute__((ext_vector_type(4)));
            const i32x2 t = __builtin_bit_cast(
                i32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)pa));
            v[2 * hh] = t[0];
            v[2 * hh + 1] = t[1];
          }
          *reinterpret_cast<i32x4*>(dst + (col0 + t0 + j) * ce.lddt + row0 + r0) = v;
        }
      };
      tstore(dgp, ce.dgt);
      tstore(dup, ce.dut);
    }
    return;
  }
  if constexpr ((EPI == 0 || EPI == 4) && EVEN && O::vec == 8) {
    if (!accumulate && vec_store == 2) {
      constexpr auto NC = std::integral_constant<int, TNW>{};
      __syncthreads();  // every wave is done with the operand ring
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          stage(NC, i, j, pack2<O>(alpha * acc[i][j][0], alpha * acc[i][j][1]),
                pack2<O>(alpha * acc[i][j][2], alpha * acc[i][j][3]));
      if (ce.res) {
        // C = res + round(acc): the residual rows of this wave's block are loaded (all 16 row passes in
        // flight) while the staging writes land, then added in fp32 to the rounded GEMM output and
        // rounded again -- exactly a GEMM output followed by q3_add.
        constexpr int CH = TNW / 8, RPI = 64 / CH;
        const int c = lane % CH;
        const u16* rsrc = ce.res + (int64_t)(m0 + wm * TMW) * ce.ldres + n0 + wn * TNW + c * 8;
        i32x4 rv[TMW / RPI];
#pragma unroll
        for (int q = 0; q < TMW / RPI; ++q)
          rv[q] = *reinterpret_cast<const i32x4*>(rsrc + (int64_t)(q * RPI + lane / CH) * ce.ldres);
        __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // this wave's staging writes
        __builtin_amdgcn_wave_barrier();
        typename O::storage* dst = C + (int64_t)(m0 + wm * TMW) * ldc + n0 + wn * TNW + c * 8;
#pragma unroll
        for (int q = 0; q < TMW / RPI; ++q) {
          const int r = q * RPI + lane / CH;
          const int sw = CH == 16 ? (r & 15) : ((r >> 1) & 7);  // the staging swizzle
          const Vec<O> a = unpack_vec<O>(*reinterpret_cast<const i32x4*>(wl + r * (TNW * 2) + ((c ^ sw) << 4)));
          const Vec<O> b = unpack_vec<O>(rv[q]);
          i32x4 o;
#pragma unroll
          for (int w = 0; w < 4; ++w) o[w] = (int)pack2<O>(a.v[2 * w] + b.v[2 * w], a.v[2 * w + 1] + b.v[2 * w + 1]);
          *reinterpret_cast<i32x4*>(dst + (int64_t)r * ldc) = o;
        }
        return;
      }
      flush(NC, C + (int64_t)(m0 + wm * TMW) * ldc + n0 + wn * TNW, ldc, std::integral_constant<int, TMW>{});
      return;
    }
  }
  if constexpr (EPI == 1 && EVEN && O::vec == 8) {
    if (vec_store == 2) {
      constexpr auto NC = std::integral_constant<int, TNW>{};
      __syncthreads();  // every wave is done with the operand ring
      uint32_t pk[FM][FN][2];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = m0 + wm * TMW + i * 16 + (lane & 15);
        const int64_t t = ce.tgt[row];
        const float lse = ce.lse[row];
        const bool valid = t != ce.ignore && t >= 0 && t < ce.vocab;
        const float scale = valid ? (ce.up ? *ce.up : 1.f) / *ce.count : 0.f;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int col = n0 + wn * TNW + j * 16 + 4 * quarter;
          float r[4];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            r[v] = scale != 0.f ? (__expf(acc[i][j][v] - lse) - ((col + v + ce.col0 == t) ? 1.f : 0.f)) * scale : 0.f;
          pk[i][j][0] = pack2<O>(r[0], r[1]);
          pk[i][j][1] = pack2<O>(r[2], r[3]);
          stage(NC, i, j, pk[i][j][0], pk[i][j][1]);
        }
      }
      flush(NC, C + (int64_t)(m0 + wm * TMW) * ldc + n0 + wn * TNW, ldc, std::integral_constant<int, TMW>{});
      if (ce.zt) {
        // transposed block: TNW rows (columns of the tile) x TMW columns (its rows), 16-bit stores
        // into 16-byte chunks swizzled as the row-major staging of a TMW-wide block
        static_assert(TMW == 64, "transposed staging assumes 64-row wave tiles");
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int tr = j * 16 + 4 * quarter + v, tc = i * 16 + (lane & 15);
              const u16 val = (u16)(pk[i][j][v >> 1] >> (16 * (v & 1)));
              *reinterpret_cast<u16*>(wl + tr * (TMW * 2) + (((tc >> 3) ^ ((tr >> 1) & 7)) << 4) + (tc & 7) * 2) = val;
            }
        flush(std::integral_constant<int, TMW>{}, ce.zt + (int64_t)(n0 + wn * TNW) * ce.ldzt + m0 + wm * TMW, ce.ldzt,
              std::integral_constant<int, TNW>{});
      }
      return;
    }
  }
  if constexpr (EPI == 2) {
    static_assert(TNW == 128, "one statistics partial per 128 columns");
    // With the logits stored: round them; full tiles stage each 16-row group of this wave's block in
    // LDS right before that group's statistics (so a group's accumulators die before the next group's
    // temporaries are live) and flush the block at the end; other tiles store each group's logits
    // directly, also beside its statistics.
    [[maybe_unused]] constexpr auto NC = std::integral_constant<int, TNW>{};
    bool staged = false;
    if (ce.zs) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[i][j][v] = to_f32<T>(from_f32<T>(acc[i][j][v]));
      if constexpr (EVEN && O::vec == 8) {
        if (vec_store == 2) {
          __syncthreads();  // every wave is done with the operand ring
          staged = true;    // each row group is staged beside its statistics below
        }
      }
    }
    const int64_t part = ce.part0 + (n0 + wn * TNW) / 128;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      if constexpr (EVEN && O::vec == 8) {
        if (staged) {
#pragma unroll
          for (int j = 0; j < FN; ++j)
            stage(NC, i, j, pack2<T>(acc[i][j][0], acc[i][j][1]), pack2<T>(acc[i][j][2], acc[i][j][3]));
        }
      }
      const int row = m0 + wm * TMW + i * 16 + (lane & 15);
      if (ce.zs && !staged && row < M) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int col = n0 + wn * TNW + j * 16 + 4 * quarter + v;
            if (col < N) ce.zs[(int64_t)row * ce.ldzs + col] = from_f32<T>(acc[i][j][v]);
          }
      }
      const int64_t t = row < M ? ce.tgt[row] - ce.col0 : -1;  // target column within this chunk
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (EVEN || n0 + wn * TNW + j * 16 + 4 * quarter + v < N) mx = fmaxf(mx, acc[i][j][v]);
      float sm = 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int col = n0 + wn * TNW + j * 16 + 4 * quarter + v;
          if (EVEN || col < N) {
            sm += mx == -INFINITY ? 0.f : __expf(acc[i][j][v] - mx);
            if (col == t) ce.pick[row] = acc[i][j][v];
          }
        }
      // the four lanes of a row (quarters) hold 32 columns each
#pragma unroll
      for (int o = 16; o < 64; o <<= 1) lse_merge(mx, sm, __shfl_xor(mx, o, 64), __shfl_xor(sm, o, 64));
      // a group that starts past N (the second half of a ragged last tile) has no partial slot
      if (quarter == 0 && row < M && n0 + wn * TNW < N) {
        ce.m_part[part * ce.ldp + row] = mx;
        ce.s_part[part * ce.ldp + row] = sm;
      }
    }
    if constexpr (EVEN && O::vec == 8) {
      if (staged)
        flush(NC, ce.zs + (int64_t)(m0 + wm * TMW) * ce.ldzs + n0 + wn * TNW, ce.ldzs,
              std::integral_constant<int, TMW>{});
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int row = m0 + wm * TMW + i * 16 + (lane & 15);
    if (row >= M) continue;
    typename O::storage* crow = C + (int64_t)row * ldc;
    [[maybe_unused]] int64_t t = 0;
    [[maybe_unused]] float lse = 0.f, scale = 0.f;
    if constexpr (EPI == 1) {
      t = ce.tgt[row];
      lse = ce.lse[row];
      const bool valid = t != ce.ignore && t >= 0 && t < ce.vocab;
      scale = valid ? (ce.up ? *ce.up : 1.f) / *ce.count : 0.f;
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn * TNW + j * 16 + 4 * quarter;
      float r[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if constexpr (EPI == 1)
          r[v] = scale != 0.f ? (__expf(acc[i][j][v] - lse) - ((col + v + ce.col0 == t) ? 1.f : 0.f)) * scale : 0.f;
        else
          r[v] = alpha * acc[i][j][v];
      }
      if (vec_store && col + 3 < N) {
        if constexpr (O::vec == 4) {
          f32x4* p = reinterpret_cast<f32x4*>(crow + col);
          if (accumulate) {
            const f32x4 o = *p;
#pragma unroll
            for (int v = 0; v < 4; ++v) r[v] += o[v];
          }
          *p = f32x4{r[0], r[1], r[2], r[3]};
        } else {
          typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
          i32x2* p = reinterpret_cast<i32x2*>(crow + col);
          if (accumulate) {
            const i32x2 o = *p;
            r[0] += to_f32<O>((u16)(o[0] & 0xffff));
            r[1] += to_f32<O>((u16)((uint32_t)o[0] >> 16));
            r[2] += to_f32<O>((u16)(o[1] & 0xffff));
            r[3] += to_f32<O>((u16)((uint32_t)o[1] >> 16));
          }
          *p = i32x2{(int)pack2<O>(r[0], r[1]), (int)pack2<O>(r[2], r[3])};
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (col + v < N) {
            float x = r[v];
            if (accumulate) x += to_f32<O>(crow[col + v]);
            crow[col + v] = from_f32<O>(x);
          }
      }
    }
  }
}

template <typename T, typename O, int BM, int BN, int WM, int WN, int ST, bool EVEN, int BK = 64, int EPI = 0>
int launch_v4(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t M, int64_t N,
              int64_t K, float alpha, int acc, hipStream_t s, CeEpi ce = CeEpi{}, int splits = 1) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  static_assert(BM * BN * 2 <= ST * (BM + BN) * BK * 2, "the LDS epilogue reuses the operand ring");
  // 2: 16-byte row stores (the LDS epilogue), 1: 8-byte (16-bit) / 16-byte (fp32) stores, 0: scalar
  const int vec = (ldc % 8 == 0 && ((uintptr_t)C & 15) == 0) ? 2
                  : ((ldc % 4 == 0) && (((uintptr_t)C & (O::vec == 4 ? 15 : 7)) == 0)) ? 1 : 0;
  gemm_nt_v4_kernel<T, O, BM, BN, WM, WN, BK, ST, EVEN, EPI><<<dim3((unsigned)tiles, (unsigned)splits), WM * WN * 64, 0, s>>>(
      (const u16*)A, (const u16*)B, (typename O::storage*)C, (int)M, (int)N, (int)K, lda, ldb, ldc, alpha, acc, vec,
      ce);
  return (int)hipGetLastError();
}

// 256 x 256 tiles (128 columns per wave) with the cross-entropy statistics epilogue.
template <typename T>
int launch_ce_stats(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                    const CeEpi& ce, hipStream_t s) {
  if (M % 256 == 0 && N % 256 == 0)
    return launch_v4<T, T, 256, 256, 4, 2, 2, true, 64, 2>(A, lda, B, ldb, nullptr, N, M, N, K, 1.f, 0, s, ce);
  return launch_v4<T, T, 256, 256, 4, 2, 2, false, 64, 2>(A, lda, B, ldb, nullptr, N, M, N, K, 1.f, 0, s, ce);
}

// Tile choice of launch_nt's K % 64 == 0 path, with the cross-entropy gradient epilogue.
template <typename T>
int launch_ce_grad(const void* A, int64_t lda, const void* B, int64_t ldb, void* dz, int64_t lddz, int64_t M,
                   int64_t N, int64_t K, const CeEpi& ce, hipStream_t s) {
  if (((M + 255) / 256) * ((N + 255) / 256) >= 256) {
    if (M % 256 == 0 && N % 256 == 0)
      return launch_v4<T, T, 256, 256, 4, 2, 2, true, 64, 1>(A, lda, B, ldb, dz, lddz, M, N, K, 1.f, 0, s, ce);
    return launch_v4<T, T, 256, 256, 4, 2, 2, false, 64, 1>(A, lda, B, ldb, dz, lddz, M, N, K, 1.f, 0, s, ce);
  }
  return launch_v4<T, T, 128, 128, 2, 2, 4, false, 64, 1>(A, lda, B, ldb, dz, lddz, M, N, K, 1.f, 0, s, ce);
}

// Gate/up GEMM with the SwiGLU epilogue: 256 x 256 tiles of the interleaved [Wg; Wu] operand, so a
// tile covers 256 rows x 128 output columns (M % 256 == 0, N % 128 == 0).
template <typename T>
int launch_gate_up(const void* X, int64_t ldx, const void* Wg, const void* Wu, int64_t ldw, void* G, void* U, void* Y,
                   int64_t ldo, int64_t M, int64_t N, int64_t K, hipStream_t s, void* Yt = nullptr, int64_t ldyt = 0) {
  CeEpi e{};
  e.b2 = (const u16*)Wu;
  e.g_out = (u16*)G;
  e.u_out = (u16*)U;
  e.yt = (u16*)Yt;
  e.ldyt = ldyt;
  return launch_v4<T, T, 256, 256, 4, 2, 2, true, 64, 3>(X, ldx, Wg, ldw, Y, ldo, M, 2 * N, K, 1.f, 0, s, e);
}

// dY = A B^T with the SwiGLU-backward epilogue (full 256 x 256 tiles only).
template <typename T>
int launch_swiglu_bwd(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                      const CeEpi& e, hipStream_t s) {
  return launch_v4<T, T, 256, 256, 4, 2, 2, true, 64, 5>(A, lda, B, ldb, e.dgo, e.lddgu, M, N, K, 1.f, 0, s, e);
}

// Q/K/V-style GEMM: one A, up to 3 weights side by side as the B rows, one output per weight
// (256 x 256 tiles of full tiles only).
int64_t tiles_of(int64_t M, int64_t N, int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }
// 256 x 256 tiles when their grid occupies at least three quarters of the 256 CUs, else 128 x 128 (two
// workgroups per CU).  Measured on MI355X: 2048 x 6144 x 4096 (192 tiles) 92.6 us against 108.0 us on
// 768 tiles of 128 x 128 (1.5 rounds); at 128 or 144 tiles of 256 x 256, 128 x 128 is faster.
bool tiles_256(int64_t M, int64_t N) { return tiles_of(M, N, 256, 256) >= 192; }
bool all_n_multiple(const int64_t* Ns, int nseg, int64_t q) {
  for (int i = 0; i < nseg; ++i)
    if (Ns[i] % q != 0) return false;
  return true;
}

template <typename T>
int launch_multi(const void* A, int64_t lda, int nseg, const void* const* Bs, int64_t ldb, void* const* Cs,
                 const int64_t* Ns, const int64_t* ldcs, int64_t M, int64_t K, hipStream_t s) {
  CeEpi e{};
  int64_t n = 0;
  for (int i = 0; i < nseg; ++i) {
    e.seg_b[i] = (const u16*)Bs[i];
    e.seg_c[i] = (u16*)Cs[i];
    e.seg_ldc[i] = ldcs[i];
    e.seg_n0[i] = n;
    n += Ns[i];
  }
  e.nseg = nseg;
  // The tile plan of the plain GEMM (the same per-element k order either way: every output equals its
  // single-weight GEMM bit for bit).
  if (M % 256 == 0 && n % 256 == 0 && tiles_256(M, n) && all_n_multiple(Ns, nseg, 256))
    return launch_v4<T, T, 256, 256, 4, 2, 2, true, 64, 4>(A, lda, Bs[0], ldb, Cs[0], ldcs[0], M, n, K, 1.f, 0, s, e);
  return launch_v4<T, T, 128, 128, 4, 2, 2, true, 64, 4>(A, lda, Bs[0], ldb, Cs[0], ldcs[0], M, n, K, 1.f, 0, s, e);
}

// ---------------------------------------------------------------- strided SIMT fallback
// C[m,n] = alpha * sum_k A[m*sam + k*sak] * B[k*sbk + n*sbn] (+ C).  64x64 tile, 4x4 per thread.
template <typename T, typename O>
__global__ __launch_bounds__(kThreads) void gemm_generic_kernel(const typename T::storage* __restrict__ A, int64_t sam,
                                                                int64_t sak, const typename T::storage* __restrict__ B,
                                                                int64_t sbk, int64_t sbn,
                                                                typename O::storage* __restrict__ C, int64_t ldc,
                                                                int M, int N, int K, float alpha, int accumulate) {
  __shared__ float As[16][65], Bs[16][65];
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int e = threadIdx.x; e < 16 * 64; e += kThreads) {
      const int kk = e / 64, mm = e % 64;
      const int gm = m0 + mm, gk = k0 + kk, gn = n0 + mm;
      As[kk][mm] = (gm < M && gk < K) ? to_f32<T>(A[(int64_t)gm * sam + (int64_t)gk * sak]) : 0.f;
      Bs[kk][mm] = (gn < N && gk < K) ? to_f32<T>(B[(int64_t)gk * sbk + (int64_t)gn * sbn]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += As[kk][ty * 4 + i] * Bs[kk][tx * 4 + j];
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m < M && n < N) {
        typename O::storage* c = C + (int64_t)m * ldc + n;
        float r = alpha * acc[i][j];
        if (accumulate) r += to_f32<O>(*c);
        *c = from_f32<O>(r);
      }
    }
}

constexpr int kBM = 256, kBN = 128, kBK = 64;


template <typename T, typename O>
int launch_nt(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t M, int64_t N,
              int64_t K, float alpha, int acc, hipStream_t s) {
  if (K % 64 == 0) {
    // 256 x 256 tiles when they fill at least three quarters of the CUs, else 128 x 128 (measured on
    // MI355X for the Qwen3-8B projection shapes: at 128 tiles of 256 x 256, 128 x 128 beats both
    // 256 x 256 and 256 x 128, e.g. 2048 x 4096 x 12288 in 190 us against 250 / 203 us).
    const int64_t t256 = tiles_of(M, N, 256, 256), nN = (N + 255) / 256;
    // A last round of 256 x 256 tiles that would leave at least half of the CUs idle (e.g. the
    // 6144 x 4096 Q/K/V weight gradient: 384 tiles) is split off along M: the rows that fill whole
    // rounds run as 256 x 256 tiles, the remaining rows as 128 x 128 tiles in a second launch
    // (same per-element k order, so the result is bit-identical to one launch).
    if (t256 > 256 && t256 % 256 != 0 && t256 % 256 <= 128 && 256 % nN == 0) {
      const int64_t m1 = (t256 / 256) * 256 / nN * 256;
      if (m1 > 0 && m1 < M) {
        const int rc = launch_nt<T, O>(A, lda, B, ldb, C, ldc, m1, N, K, alpha, acc, s);
        if (rc != 0) return rc;
        return launch_nt<T, O>(static_cast<const u16*>(A) + m1 * lda, lda, B, ldb,
                               static_cast<typename O::storage*>(C) + m1 * ldc, ldc, M - m1, N, K, alpha, acc, s);
      }
    }
    if (tiles_256(M, N)) {
      if (M % 256 == 0 && N % 256 == 0)
        return launch_v4<T, O, 256, 256, 4, 2, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
      return launch_v4<T, O, 256, 256, 4, 2, 2, false>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
    }
    // 128 x 128 tiles: 8 waves of 32 x 64 over a 2-stage ring (64 KB of LDS: two workgroups per CU).
    // Measured on the prefill-size shapes (M = 1024 / 2048 / 4096): 615-629 us in total against 666-673
    // for 4 waves of 64 x 64 over 4 stages (one workgroup per CU) and 648 for 8 waves over 3 stages.
    if (M % 128 == 0 && N % 128 == 0)
      return launch_v4<T, O, 128, 128, 4, 2, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
    return launch_v4<T, O, 128, 128, 2, 2, 4, false>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
  }
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  gemm_nt_kernel<T, O, kBM, kBN, kBK, 128, 64><<<(unsigned)tiles, kThreads, 0, s>>>(
      (const u16*)A, (const u16*)B, (typename O::storage*)C, (int)M, (int)N, (int)K, lda, ldb, ldc, alpha, acc);
  return (int)hipGetLastError();
}

template <typename T>
int nt_out(int out, const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t M,
           int64_t N, int64_t K, float alpha, int acc, hipStream_t s) {
  if (out == Q3_F32) return launch_nt<T, F32>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
  if (out == Q3_F16) return launch_nt<T, F16>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
  return launch_nt<T, BF16>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
}

template <typename T, typename O>
int launch_generic(const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk, int64_t sbn, void* C,
                   int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha, int acc, hipStream_t s) {
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  gemm_generic_kernel<T, O><<<grid, kThreads, 0, s>>>((const typename T::storage*)A, sam, sak,
                                                      (const typename T::storage*)B, sbk, sbn,
                                                      (typename O::storage*)C, ldc, (int)M, (int)N, (int)K, alpha,
                                                      acc);
  return (int)hipGetLastError();
}

template <typename T>
int generic_out(int out, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk, int64_t sbn, void* C,
                int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha, int acc, hipStream_t s) {
  if (out == Q3_F32) return launch_generic<T, F32>(A, sam, sak, B, sbk, sbn, C, ldc, M, N, K, alpha, acc, s);
  if (out == Q3_F16) return launch_generic<T, F16>(A, sam, sak, B, sbk, sbn, C, ldc, M, N, K, alpha, acc, s);
  return launch_generic<T, BF16>(A, sam, sak, B, sbk, sbn, C, ldc, M, N, K, alpha, acc, s);
}

bool dtype_ok(int dt) { return dt == Q3_F32 || dt == Q3_F16 || dt == Q3_BF16; }
bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }


// Residual GEMM as two K splits (at least kSplitKMin of K each): 256 x 256 tiles whose grid alone would
// occupy at most half of the 256 CUs (and so runs as 128 x 128 tiles otherwise) doubled along K.
// Measured on MI355X at M = 2048, N = 4096: K = 12288 161 + 16 us (the combining pass) against 207 us on
// 128 x 128 tiles; K = 4096 65 + 16 against 69 us, hence the minimum.
constexpr int64_t kSplitKMin = 4096;
int residual_splits(int64_t M, int64_t N, int64_t K) {
  if (M % 256 != 0 || N % 256 != 0 || K % 128 != 0 || K / 2 < kSplitKMin) return 1;
  const int64_t t = tiles_of(M, N, 256, 256);
  return t >= 96 && t <= 128 ? 2 : 1;
}

// C = R + (P0 + P1) from the two fp32 partial products (P1 at P0 + split_ld, row stride N) with the
// roundings of the unsplit residual GEMM: the product rounded to T, added to R in fp32, rounded again.
template <typename T>
__global__ __launch_bounds__(256) void split_residual_kernel(const float* __restrict__ P, int64_t split_ld,
                                                             const u16* __restrict__ R, int64_t ldr,
                                                             u16* __restrict__ C, int64_t ldc, int64_t M, int64_t N) {
  const int64_t cols = N / 8, i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * cols) return;
  const int64_t r = i / cols, c = (i - r * cols) * 8;
  const float* p = P + r * N + c;
  const f32x4 a0 = *reinterpret_cast<const f32x4*>(p), a1 = *reinterpret_cast<const f32x4*>(p + 4);
  const f32x4 b0 = *reinterpret_cast<const f32x4*>(p + split_ld), b1 = *reinterpret_cast<const f32x4*>(p + split_ld + 4);
  const i32x4 rv = *reinterpret_cast<const i32x4*>(R + r * ldr + c);
  i32x4 o;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float s0 = w < 2 ? a0[2 * w] + b0[2 * w] : a1[2 * w - 4] + b1[2 * w - 4];
    const float s1 = w < 2 ? a0[2 * w + 1] + b0[2 * w + 1] : a1[2 * w - 3] + b1[2 * w - 3];
    const u16 lo = from_f32<T>(to_f32<T>(from_f32<T>(s0)) + to_f32<T>((u16)(rv[w] & 0xffff)));
    const u16 hi = from_f32<T>(to_f32<T>(from_f32<T>(s1)) + to_f32<T>((u16)((uint32_t)rv[w] >> 16)));
    o[w] = (int)((uint32_t)lo | ((uint32_t)hi << 16));
  }
  *reinterpret_cast<i32x4*>(C + r * ldc + c) = o;
}

// split_residual_kernel's C for one row per 512-thread workgroup, and also Y = C rsqrt(mean(C^2) + eps) w
// (the following RMSNorm, from the rounded C: q3_rmsnorm_fwd's expression, one rounding).
template <typename T>
__global__ __launch_bounds__(512) void split_residual_norm_kernel(const float* __restrict__ P, int64_t split_ld,
                                                                  const u16* __restrict__ R, int64_t ldr,
                                                                  u16* __restrict__ C, int64_t ldc,
                                                                  const u16* __restrict__ w, float eps,
                                                                  u16* __restrict__ Y, int64_t ldy, int N) {
  constexpr int kMaxG = 2;  // 8-column groups per thread: N <= 8192
  __shared__ float red[8];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  float c[kMaxG][8];
  float ss = 0.f;
#pragma unroll
  for (int gi = 0; gi < kMaxG; ++gi) {
    const int col = (gi * 512 + tid) * 8;
    if (col < N) {
      const float* p = P + r * N + col;
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(p), a1 = *reinterpret_cast<const f32x4*>(p + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(p + split_ld);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(p + split_ld + 4);
      const i32x4 rv = *reinterpret_cast<const i32x4*>(R + r * ldr + col);
      i32x4 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sum = e < 4 ? a0[e] + b0[e] : a1[e - 4] + b1[e - 4];
        const u16 rr = (u16)(((uint32_t)rv[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        c[gi][e] = to_f32<T>(from_f32<T>(to_f32<T>(from_f32<T>(sum)) + to_f32<T>(rr)));
        ss += c[gi][e] * c[gi][e];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = (int)pack2<T>(c[gi][2 * q], c[gi][2 * q + 1]);
      *reinterpret_cast<i32x4*>(C + r * ldc + col) = o;
    }
  }
  ss = group_sum<64>(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) tot += red[i];
  const float inv = rsqrtf(tot * (1.f / (float)N) + eps);
#pragma unroll
  for (int gi = 0; gi < kMaxG; ++gi) {
    const int col = (gi * 512 + tid) * 8;
    if (col < N) {
      const i32x4 wv = *reinterpret_cast<const i32x4*>(w + col);
      i32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float w0 = to_f32<T>((u16)((uint32_t)wv[q] & 0xffffu)), w1 = to_f32<T>((u16)((uint32_t)wv[q] >> 16));
        o[q] = (int)pack2<T>(c[gi][2 * q] * inv * w0, c[gi][2 * q + 1] * inv * w1);
      }
      *reinterpret_cast<i32x4*>(Y + r * ldy + col) = o;
    }
  }
}

template <typename T>
int launch_split_residual(const void* A, int64_t lda, const void* B, int64_t ldb, const void* R, int64_t ldr,
                          void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, float* P, hipStream_t s,
                          const void* nw = nullptr, float eps = 0.f, void* Y = nullptr, int64_t ldy = 0) {
  CeEpi e{};
  e.split_ld = M * N;
  int rc = launch_v4<T, F32, 256, 256, 4, 2, 2, true>(A, lda, B, ldb, P, N, M, N, K, 1.f, 0, s, e, 2);
  if (rc != 0) return rc;
  if (Y) {
    split_residual_norm_kernel<T><<<(unsigned)M, 512, 0, s>>>(P, M * N, (const u16*)R, ldr, (u16*)C, ldc,
                                                              (const u16*)nw, eps, (u16*)Y, ldy, (int)N);
    return (int)hipGetLastError();
  }
  const int64_t n8 = M * N / 8;
  split_residual_kernel<T><<<(unsigned)((n8 + 255) / 256), 256, 0, s>>>(P, M * N, (const u16*)R, ldr, (u16*)C, ldc,
                                                                        M, N);
  return (int)hipGetLastError();
}

}  // namespace

// Tuning hook (not part of the public ABI header): runs one fixed tile variant of the bf16 NT GEMM
// with bf16 output, so configurations can be timed side by side.
extern "C" int q3_gemm_nt_variant(int variant, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
                                  int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  switch (variant) {
    case 0: return launch_v4<BF16, BF16, 256, 256, 4, 2, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 1: return launch_v4<BF16, BF16, 256, 256, 2, 4, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 2: return launch_v4<BF16, BF16, 256, 256, 4, 2, 2, false>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 3: return launch_v4<BF16, BF16, 256, 128, 2, 2, 3, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 4: return launch_v4<BF16, BF16, 128, 128, 2, 2, 4, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 5: return launch_v4<BF16, BF16, 256, 256, 4, 2, 4, true, 32>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 6: return launch_v4<BF16, BF16, 256, 256, 4, 2, 5, true, 32>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 7: return launch_v4<BF16, BF16, 256, 256, 2, 4, 4, true, 32>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 8: return launch_v4<BF16, BF16, 256, 128, 2, 2, 6, true, 32>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 9: return launch_v4<BF16, BF16, 128, 128, 2, 2, 8, true, 32>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    default: return Q3_ERR_INVALID;
  }
}

extern "C" {

int q3_gemm_nt(int in_dtype, int out_dtype, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
               int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha, int accumulate, hipStream_t stream) {
  Q3_REQUIRE((in_dtype == Q3_BF16 || in_dtype == Q3_F16) && dtype_ok(out_dtype) && A && B && C);
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31));
  Q3_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K && ldc >= N && al16(A) && al16(B));
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  Q3_REQUIRE(tiles < (1ll << 31));
  if (in_dtype == Q3_BF16) return nt_out<BF16>(out_dtype, A, lda, B, ldb, C, ldc, M, N, K, alpha, accumulate, stream);
  return nt_out<F16>(out_dtype, A, lda, B, ldb, C, ldc, M, N, K, alpha, accumulate, stream);
}

int q3_gemm_nt_ce_grad(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, void* dz, int64_t lddz,
                       void* dzt, int64_t lddzt, int64_t M, int64_t N, int64_t K, int64_t col0, const int64_t* tgt,
                       const float* lse, const float* count, const float* up, int64_t vocab, int64_t ignore_index,
                       hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && A && B && dz && tgt && lse && count);
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && K % 64 == 0);
  Q3_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K && lddz >= N && al16(A) && al16(B));
  // the transposed copy comes from the LDS epilogue of full 256 x 256 tiles with 16-byte row stores
  Q3_REQUIRE(!dzt || (M % 256 == 0 && N % 256 == 0 && (M / 256) * (N / 256) >= 256 && lddz % 8 == 0 && al16(dz) &&
                      lddzt % 8 == 0 && lddzt >= M && al16(dzt)));
  CeEpi ce{tgt, lse, count, up, col0, vocab, ignore_index, nullptr, nullptr, nullptr, 0, 0};
  ce.zt = (u16*)dzt;
  ce.ldzt = lddzt;
  if (dtype == Q3_BF16) return launch_ce_grad<BF16>(A, lda, B, ldb, dz, lddz, M, N, K, ce, stream);
  return launch_ce_grad<F16>(A, lda, B, ldb, dz, lddz, M, N, K, ce, stream);
}

int q3_gemm_nt_ce_stats(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                        int64_t K, int64_t col0, const int64_t* tgt, float* m_part, float* s_part, float* pick,
                        int64_t part0, int64_t ldp, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && A && B && tgt && m_part && s_part && pick);
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && K % 64 == 0);
  Q3_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K && ldp >= M && part0 >= 0 && al16(A) && al16(B));
  const CeEpi ce{tgt, nullptr, nullptr, nullptr, col0, 0, 0, m_part, s_part, pick, part0, ldp};
  if (dtype == Q3_BF16) return launch_ce_stats<BF16>(A, lda, B, ldb, M, N, K, ce, stream);
  return launch_ce_stats<F16>(A, lda, B, ldb, M, N, K, ce, stream);
}

int q3_gemm_nt_ce_stats_store(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                              int64_t K, int64_t col0, const int64_t* tgt, float* m_part, float* s_part, float* pick,
                              int64_t part0, int64_t ldp, void* z, int64_t ldz, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && A && B && tgt && m_part && s_part && pick && z);
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && K % 64 == 0);
  Q3_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K && ldp >= M && part0 >= 0 && al16(A) && al16(B));
  Q3_REQUIRE(ldz >= N && ldz % 8 == 0 && al16(z));
  CeEpi ce{tgt, nullptr, nullptr, nullptr, col0, 0, 0, m_part, s_part, pick, part0, ldp};
  ce.zs = (u16*)z;
  ce.ldzs = ldz;
  if (dtype == Q3_BF16) return launch_ce_stats<BF16>(A, lda, B, ldb, M, N, K, ce, stream);
  return launch_ce_stats<F16>(A, lda, B, ldb, M, N, K, ce, stream);
}

int q3_gemm_gate_up_swiglu(int dtype, const void* x, int64_t ldx, const void* wg, const void* wu, int64_t ldw,
                           void* g, void* u, void* y, int64_t ldo, int64_t M, int64_t N, int64_t K,
                           hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && x && wg && wu && !g == !u && y);
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M % 256 == 0 && N % 128 == 0 && K % 64 == 0 && M < (1ll << 31) &&
             N < (1ll << 30) && K < (1ll << 31) && (M / 256) * (N / 128) < (1ll << 31));
  Q3_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0 && ldo % 8 == 0 && ldx >= K && ldw >= K && ldo >= N && al16(x) &&
             al16(wg) && al16(wu) && al16(g) && al16(u) && al16(y));
  if (dtype == Q3_BF16) return launch_gate_up<BF16>(x, ldx, wg, wu, ldw, g, u, y, ldo, M, N, K, stream);
  return launch_gate_up<F16>(x, ldx, wg, wu, ldw, g, u, y, ldo, M, N, K, stream);
}

int q3_gemm_gate_up_swiglu_t(int dtype, const void* x, int64_t ldx, const void* wg, const void* wu, int64_t ldw,
                             void* g, void* u, void* y, int64_t ldo, void* yt, int64_t ldyt, int64_t M, int64_t N,
                             int64_t K, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && x && wg && wu && g && u && y && yt);
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M % 256 == 0 && N % 128 == 0 && K % 64 == 0 && M < (1ll << 31) &&
             N < (1ll << 30) && K < (1ll << 31) && (M / 256) * (N / 128) < (1ll << 31));
  Q3_REQUIRE(ldx % 8 == 0 && ldw % 8 == 0 && ldo % 8 == 0 && ldx >= K && ldw >= K && ldo >= N && al16(x) &&
             al16(wg) && al16(wu) && al16(g) && al16(u) && al16(y));
  Q3_REQUIRE(ldyt % 8 == 0 && ldyt >= M && al16(yt));
  if (dtype == Q3_BF16) return launch_gate_up<BF16>(x, ldx, wg, wu, ldw, g, u, y, ldo, M, N, K, stream, yt, ldyt);
  return launch_gate_up<F16>(x, ldx, wg, wu, ldw, g, u, y, ldo, M, N, K, stream, yt, ldyt);
}

size_t q3_gemm_nt_residual_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && residual_splits(M, N, K) > 1 ? (size_t)(2 * M * N) * sizeof(float) : 0;
}

int q3_gemm_nt_residual_ws(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, const void* R,
                           int64_t ldr, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && A && B && R && C);
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M % 128 == 0 && N % 128 == 0 && K % 64 == 0 && M < (1ll << 31) &&
             N < (1ll << 31) && K < (1ll << 31) && (M / 128) * (N / 128) < (1ll << 31));
  Q3_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && ldr % 8 == 0 && ldc % 8 == 0 && lda >= K && ldb >= K && ldr >= N &&
             ldc >= N && al16(A) && al16(B) && al16(R) && al16(C));
  const size_t need = q3_gemm_nt_residual_workspace_bytes(M, N, K);
  if (need > 0 && workspace) {
    Q3_REQUIRE(workspace_bytes >= need && al16(workspace));
    if (dtype == Q3_BF16)
      return launch_split_residual<BF16>(A, lda, B, ldb, R, ldr, C, ldc, M, N, K, (float*)workspace, stream);
    return launch_split_residual<F16>(A, lda, B, ldb, R, ldr, C, ldc, M, N, K, (float*)workspace, stream);
  }
  CeEpi e{};
  e.res = (const u16*)R;
  e.ldres = ldr;
  // The plain GEMM's tile plan.
  const bool big = M % 256 == 0 && N % 256 == 0 && tiles_256(M, N);
  if (dtype == Q3_BF16) {
    if (big) return launch_v4<BF16, BF16, 256, 256, 4, 2, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, stream, e);
    return launch_v4<BF16, BF16, 128, 128, 4, 2, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, stream, e);
  }
  if (big) return launch_v4<F16, F16, 256, 256, 4, 2, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, stream, e);
  return launch_v4<F16, F16, 128, 128, 4, 2, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, stream, e);
}

int q3_gemm_nt_residual(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, const void* R,
                        int64_t ldr, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  return q3_gemm_nt_residual_ws(dtype, A, lda, B, ldb, R, ldr, C, ldc, M, N, K, nullptr, 0, stream);
}

int q3_gemm_nt_residual_norm_ws(int dtype, const void* A, int64_t lda, const void* B, int64_t ldb, const void* R,
                                int64_t ldr, void* C, int64_t ldc, const void* norm_w, float eps, void* Y,
                                int64_t ldy, int64_t M, int64_t N, int64_t K, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  Q3_REQUIRE(norm_w && Y && eps > 0.f && N <= 8192 && ldy % 8 == 0 && ldy >= N && al16(norm_w) && al16(Y));
  const size_t need = q3_gemm_nt_residual_workspace_bytes(M, N, K);
  if (need == 0 || !workspace) {  // the residual GEMM, then the norm as its own pass
    const int rc = q3_gemm_nt_residual_ws(dtype, A, lda, B, ldb, R, ldr, C, ldc, M, N, K, nullptr, 0, stream);
    if (rc != 0) return rc;
    Q3_REQUIRE(ldc == N && ldy == N);
    return q3_rmsnorm_fwd(dtype, C, norm_w, Y, M, N, eps, stream);
  }
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && A && B && R && C && workspace_bytes >= need &&
             al16(workspace));
  Q3_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && ldr % 8 == 0 && ldc % 8 == 0 && lda >= K && ldb >= K && ldr >= N &&
             ldc >= N && al16(A) && al16(B) && al16(R) && al16(C));
  if (dtype == Q3_BF16)
    return launch_split_residual<BF16>(A, lda, B, ldb, R, ldr, C, ldc, M, N, K, (float*)workspace, stream, norm_w,
                                       eps, Y, ldy);
  return launch_split_residual<F16>(A, lda, B, ldb, R, ldr, C, ldc, M, N, K, (float*)workspace, stream, norm_w, eps,
                                    Y, ldy);
}

int q3_gemm_swiglu_bwd(int dtype, const void* dy, int64_t lddy, const void* wt, int64_t ldw, const void* g,
                       const void* u, int64_t ldgu, void* dg, void* du, int64_t ldd, void* dgt, void* dut,
                       int64_t lddt, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && dy && wt && g && u && dg && du && (!dgt == !dut));
  Q3_REQUIRE(M > 0 && N > 0 && K > 0 && M % 256 == 0 && N % 256 == 0 && K % 64 == 0 && M < (1ll << 31) &&
             N < (1ll << 31) && K < (1ll << 31) && (M / 256) * (N / 256) < (1ll << 31));
  Q3_REQUIRE(lddy % 8 == 0 && ldw % 8 == 0 && ldgu % 8 == 0 && ldd % 8 == 0 && lddy >= K && ldw >= K &&
             ldgu >= N && ldd >= N && al16(dy) && al16(wt) && al16(g) && al16(u) && al16(dg) && al16(du));
  Q3_REQUIRE(!dgt || (lddt % 8 == 0 && lddt >= M && al16(dgt) && al16(dut)));
  CeEpi e{};
  e.gin = (const u16*)g;
  e.uin = (const u16*)u;
  e.ldgu = ldgu;
  e.dgo = (u16*)dg;
  e.duo = (u16*)du;
  e.lddgu = ldd;
  e.dgt = (u16*)dgt;
  e.dut = (u16*)dut;
  e.lddt = lddt;
  if (dtype == Q3_BF16) return launch_swiglu_bwd<BF16>(dy, lddy, wt, ldw, M, N, K, e, stream);
  return launch_swiglu_bwd<F16>(dy, lddy, wt, ldw, M, N, K, e, stream);
}

int q3_gemm_nt_multi(int dtype, const void* A, int64_t lda, int nseg, const void* const* Bs, int64_t ldb,
                     void* const* Cs, const int64_t* Ns, const int64_t* ldcs, int64_t M, int64_t K,
                     hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && A && Bs && Cs && Ns && ldcs && nseg >= 1 && nseg <= 3);
  Q3_REQUIRE(M > 0 && K > 0 && M % 128 == 0 && K % 64 == 0 && M < (1ll << 31) && K < (1ll << 31));
  Q3_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K && al16(A));
  int64_t n = 0;
  for (int i = 0; i < nseg; ++i) {
    Q3_REQUIRE(Bs[i] && Cs[i] && Ns[i] > 0 && Ns[i] % 128 == 0 && ldcs[i] >= Ns[i] && ldcs[i] % 8 == 0 &&
               al16(Bs[i]) && al16(Cs[i]));
    n += Ns[i];
  }
  Q3_REQUIRE(n < (1ll << 31) && (M / 128) * (n / 128) < (1ll << 31));
  if (dtype == Q3_BF16) return launch_multi<BF16>(A, lda, nseg, Bs, ldb, Cs, Ns, ldcs, M, K, stream);
  return launch_multi<F16>(A, lda, nseg, Bs, ldb, Cs, Ns, ldcs, M, K, stream);
}

int q3_gemm_strided(int in_dtype, int out_dtype, const void* A, int64_t sam, int64_t sak, const void* B, int64_t sbk,
                    int64_t sbn, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, float alpha, int accumulate,
                    hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(in_dtype) && dtype_ok(out_dtype) && A && B && C && M > 0 && N > 0 && K > 0);
  Q3_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && (M + 63) / 64 < 65536 && ldc >= N);
  if (in_dtype == Q3_BF16)
    return generic_out<BF16>(out_dtype, A, sam, sak, B, sbk, sbn, C, ldc, M, N, K, alpha, accumulate, stream);
  if (in_dtype == Q3_F16)
    return generic_out<F16>(out_dtype, A, sam, sak, B, sbk, sbn, C, ldc, M, N, K, alpha, accumulate, stream);
  return generic_out<F32>(out_dtype, A, sam, sak, B, sbk, sbn, C, ldc, M, N, K, alpha, accumulate, stream);
}

}  // extern "C"

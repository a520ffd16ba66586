// bf16/fp16 GEMM on CDNA4 matrix cores, plus a strided SIMT fallback.
//
// gemm_nt:  C[M,N] = alpha * A[M,K] . B[N,K]^T (+ C if accumulate), both operands K-contiguous
// (the layout of X and of a row-major weight W[N,K] in Y = X W^T).  fp32 accumulation in
// v_mfma_f32_32x32x16_{bf16,f16}; output in bf16/fp16/fp32.
//
// Tiling: workgroup tile BM x BN x BK = 256 x 128 x 64, 4 waves in a 2 x 2 grid, each wave a
// 128 x 64 sub-tile = 4 x 2 MFMA 32x32 tiles (128 fp32 accumulators per lane).  Global -> LDS
// moves 16-byte vectors (8 consecutive k) staged through registers one k-tile ahead; LDS is
// double-buffered so one barrier per k-tile suffices.  LDS rows are padded to BK+8 elements
// (144 B): the 32 rows read by one MFMA operand fetch land on distinct 4-bank groups, so every
// ds_read_b128 is conflict free.  Workgroup ids are remapped so that each XCD (ids congruent
// mod 8) owns a contiguous range of output tiles, then rastered in groups of 8 tile-rows so
// consecutive tiles share A rows in that XCD's L2.
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
  constexpr int GROUP = 8;
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

// ---------------------------------------------------------------- v2: direct-to-LDS, swizzled ring
// Same contract as gemm_nt_kernel for K % BK == 0.  Each wave-wide global_load_lds_dwordx4 moves
// 64 x 16 bytes straight into LDS (no register staging) into a ring of STAGES k-tiles, so
// STAGES-1 tiles of A and B rows are in flight while one feeds the matrix cores.  LDS rows are
// BK*2 bytes unpadded; the 16-byte chunk c of stage row R is stored at physical chunk c ^ swz(R),
// chosen so that the 8- and 16-lane groups of every MFMA operand read (32 rows, one logical chunk)
// hit distinct banks.  The lane -> global address map applies the same swizzle, because the LDS
// destination of a wave load is fixed (base + lane * 16).  Rows beyond M/N load a clamped valid row:
// they only feed output rows/columns that are never stored.
template <int CPR> Q3_DEV int lds_swz(int r) {
  if constexpr (CPR == 8) return (r ^ (r >> 3)) & 7;
  else return ((r >> 1) ^ (r >> 3)) & 3;  // 4 chunks (64-byte rows)
}

// s_waitcnt with vmcnt = N (N < 64) and lgkm/exp counters left unconstrained.
template <int N> Q3_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <typename T, typename O, int BM, int BN, int WM, int WN, int BK, int STAGES, bool PIPE = false>
__global__ __launch_bounds__(WM * WN * 64) void gemm_nt_v2_kernel(const u16* __restrict__ A,
                                                                  const u16* __restrict__ B,
                                                                  typename O::storage* __restrict__ C, int M, int N,
                                                                  int K, int64_t lda, int64_t ldb, int64_t ldc,
                                                                  float alpha, int accumulate) {
  constexpr int NW = WM * WN, ROWB = BK * 2, CPR = BK / 8, RPL = 64 / CPR;
  constexpr int TMW = BM / WM, TNW = BN / WN, TM = TMW / 32, TN = TNW / 32;
  constexpr int RG = (BM + BN) / RPL;                  // row groups per stage (one wave load each)
  static_assert(RG % NW == 0, "row groups must split evenly over the waves");
  constexpr int LPW = RG / NW;                         // wave loads per k-tile
  constexpr int STAGE = (BM + BN) * BK;                // elements per stage
  __shared__ __attribute__((aligned(1024))) u16 lds[STAGES * STAGE];

  int tm, tn;
  tile_coords(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const u16* src[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int rg = wave + NW * i;
    const int R = rg * RPL + lane / CPR;                 // row in the combined [A; B] stage
    const int c = (lane % CPR) ^ lds_swz<CPR>(R);        // logical 16-byte chunk this lane fetches
    if (R < BM) {
      src[i] = A + (int64_t)min(m0 + R, M - 1) * lda + c * 8;
    } else {
      src[i] = B + (int64_t)min(n0 + R - BM, N - 1) * ldb + c * 8;
    }
  }
  auto issue = [&](int stage, int k0) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int rg = wave + NW * i;
      __builtin_amdgcn_global_load_lds((const void*)(src[i] + k0),
                                       (__attribute__((address_space(3))) void*)(lds + stage * STAGE + rg * RPL * BK),
                                       16, 0, 0);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = K / BK;
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st)
    if (st < nk) issue(st, st * BK);
  int ra[TM], rb[TN], sa[TM], sb[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    ra[i] = wm * TMW + i * 32 + (lane & 31);
    sa[i] = lds_swz<CPR>(ra[i]);
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    rb[j] = BM + wn * TNW + j * 32 + (lane & 31);
    sb[j] = lds_swz<CPR>(rb[j]);
  }
  const int half = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    // Tile kt must have landed; the later tiles of the ring may stay in flight.
    if (nk - 1 - kt >= STAGES - 2) wait_vmcnt<(STAGES - 2) * LPW>();
    else wait_vmcnt<0>();
    __syncthreads();  // every wave's share of tile kt is in LDS; stage (kt-1) % STAGES is free
    if (kt + STAGES - 1 < nk) issue((kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK);
    const char* base = reinterpret_cast<const char*>(lds + (kt % STAGES) * STAGE);
    if constexpr (!PIPE) {
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        const int c = ks * 2 + half;
        bf16x8_t af[TM], bfr[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const bf16x8_t*>(base + ra[i] * ROWB + ((c ^ sa[i]) << 4));
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8_t*>(base + rb[j] * ROWB + ((c ^ sb[j]) << 4));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x16<T>(af[i], bfr[j], acc[i][j]);
      }
    } else {
      // Fragments double-buffered across k-steps: the reads of step ks+1 are issued before the
      // MFMAs of step ks and the scheduler is asked to interleave them one for one.
      constexpr int KS = BK / 16;
      bf16x8_t af[2][TM], bfr[2][TN];
      auto load = [&](int buf, int ks) {
        const int c = ks * 2 + half;
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[buf][i] = *reinterpret_cast<const bf16x8_t*>(base + ra[i] * ROWB + ((c ^ sa[i]) << 4));
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bfr[buf][j] = *reinterpret_cast<const bf16x8_t*>(base + rb[j] * ROWB + ((c ^ sb[j]) << 4));
      };
      load(0, 0);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) load((ks + 1) & 1, ks + 1);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x16<T>(af[ks & 1][i], bfr[ks & 1][j], acc[i][j]);
        if (ks + 1 < KS) {
#pragma unroll
          for (int x = 0; x < TM + TN; ++x) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          }
          if (TM * TN > TM + TN) __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
        } else {
          __builtin_amdgcn_sched_group_barrier(0x008, TM * TN, 0);
        }
      }
    }
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wn * TNW + j * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm * TMW + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M && col < N) {
          typename O::storage* c = C + (int64_t)row * ldc + col;
          float r = alpha * acc[i][j][v];
          if (accumulate) r += to_f32<O>(*c);
          *c = from_f32<O>(r);
        }
      }
    }
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

template <typename T, typename O, int BM, int BN, int WM, int WN, int BK = 64, int ST = 2, bool PIPE = false>
int launch_v2(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t M, int64_t N,
              int64_t K, float alpha, int acc, hipStream_t s) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  gemm_nt_v2_kernel<T, O, BM, BN, WM, WN, BK, ST, PIPE><<<(unsigned)tiles, WM * WN * 64, 0, s>>>(
      (const u16*)A, (const u16*)B, (typename O::storage*)C, (int)M, (int)N, (int)K, lda, ldb, ldc, alpha, acc);
  return (int)hipGetLastError();
}

int64_t tiles_of(int64_t M, int64_t N, int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

template <typename T, typename O>
int launch_nt(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int64_t M, int64_t N,
              int64_t K, float alpha, int acc, hipStream_t s) {
  if (K % 64 == 0) {
    // Largest tile that still gives every CU (256) a workgroup (tile choice measured on MI355X
    // for the Qwen3-8B projection shapes).
    if (tiles_of(M, N, 256, 256) >= 256)
      return launch_v2<T, O, 256, 256, 2, 4, 64, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
    if (tiles_of(M, N, 256, 128) >= 256)
      return launch_v2<T, O, 256, 128, 2, 2, 64, 3>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
    return launch_v2<T, O, 128, 128, 2, 2, 64, 4>(A, lda, B, ldb, C, ldc, M, N, K, alpha, acc, s);
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

}  // namespace

// Tuning hook (not part of the public ABI header): runs one fixed tile variant of the bf16 NT GEMM
// with bf16 output, so configurations can be timed side by side.
extern "C" int q3_gemm_nt_variant(int variant, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
                                  int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  switch (variant) {
    case 0: return launch_v2<BF16, BF16, 256, 256, 2, 4, 64, 2>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 1: return launch_v2<BF16, BF16, 256, 256, 2, 4, 32, 4>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 2: return launch_v2<BF16, BF16, 256, 128, 2, 2, 64, 3>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 3: return launch_v2<BF16, BF16, 256, 128, 2, 2, 32, 4>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 4: return launch_v2<BF16, BF16, 128, 128, 2, 2, 64, 4>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 5: return launch_v2<BF16, BF16, 256, 256, 2, 4, 32, 3>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 6: return launch_v2<BF16, BF16, 256, 256, 4, 2, 64, 2>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 7: return launch_v2<BF16, BF16, 128, 256, 2, 2, 64, 3>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 8: return launch_v2<BF16, BF16, 256, 256, 2, 4, 64, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 9: return launch_v2<BF16, BF16, 256, 256, 4, 2, 64, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 10: return launch_v2<BF16, BF16, 256, 128, 2, 2, 64, 3, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 11: return launch_v2<BF16, BF16, 128, 128, 2, 2, 64, 4, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
    case 12: return launch_v2<BF16, BF16, 256, 256, 2, 2, 64, 2, true>(A, lda, B, ldb, C, ldc, M, N, K, 1.f, 0, s);
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

// Single-GPU greedy decode: small-M GEMV, KV-cache append, split-KV decode attention and the
// greedy argmax/select step.  All four are bound by HBM traffic (weights, cache, logits).
#include <mutex>
#include <type_traits>

#include "common.h"

namespace {

constexpr int kThreads = 256;

// ============================================================================ decode linear
// y_s[m, n] = epilogue(sum_k xn[m, k] W_s[n, k]) for M <= 16 token rows (a decode step), on matrix
// cores: v_mfma_f32_16x16x32 with the token rows as the A operand (rows >= M are zero) and 16 weight
// rows as the B operand.  The weights stream straight into registers: per 128-wide k block, k-step c
// takes k in [kb + 32 c, +32) and lane l (row n = l % 16, quarter kq = l / 16) loads its 8 k at
// kb + 32 c + 8 kq, so each load instruction reads 64 contiguous bytes of 16 rows.  A workgroup owns
// 16 output rows and its NW waves take interleaved k blocks, P blocks in flight per wave (all loads
// issued before the block's MFMAs); the partial 16 x 16 tiles fold in LDS in fixed order.
//   * NORM: the RMSNorm of the input rows folded in: y = rsqrt(mean_k x[m, k]^2 + eps) *
//     sum_k T(x[m, k] norm_w[k]) W[n, k] -- the row scale multiplies the fp32 dot product, and each
//     workgroup accumulates the sums of squares from the x chunks it already streams (no separate
//     normalisation pass before the weights);
//   * MODE 0: y = acc;  MODE 1: y = res + T(acc) (residual add);  MODE 2: segments 0 and 1 are the
//     gate and up weights, y_0 = silu(T(acc_gate)) * T(acc_up) (SwiGLU);
//   * up to 3 weight segments share the input (the Q, K and V projections in one launch).
// Rounding points: the GEMV output, then residual / SwiGLU, as the unfused path (which rounds the
// normalised input before its GEMM instead); every output is a fixed-order reduction: deterministic.
struct DecSeg {
  const u16* w;
  u16* y;
  int64_t ldy;
  int n, tiles;
};
struct DecArgs {
  DecSeg seg[3];
  int nseg;
  const u16* x;
  int64_t ldx;
  int M, K;
  const u16* nw;
  float eps;
  const u16* res;
  int64_t ldres;
};

template <typename T, int MODE, bool NORM, int NW, int P>
__global__ __launch_bounds__(NW * 64) void dlinear_kernel(DecArgs a) {
  constexpr int NB = MODE == 2 ? 2 : 1;  // weight tiles per workgroup (gate + up)
  __shared__ f32x4 red[NW][NB][64];
  __shared__ float red_ss[NORM ? NW : 1][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int tile = blockIdx.x, s = 0;
  if constexpr (MODE != 2) {
    while (s + 1 < a.nseg && tile >= a.seg[s].tiles) tile -= a.seg[s++].tiles;
  }
  const DecSeg sg = a.seg[s];
  const int n0 = tile * 16, K = a.K, M = a.M;
  const int r = lane & 15, kq = lane >> 4;  // r: token row (A) and weight row (B) of this lane

  const bool xrow = r < M;
  // NORM: y = inv[m] * sum_k (x[m, k] nw[k]) W[n, k] with inv[m] = rsqrt(mean_k x[m, k]^2 + eps): the
  // per-row scale is applied after the dot product, and the sum of squares is accumulated from the
  // same x chunks the MFMAs consume, so no separate normalisation pass precedes the weight stream.
  float ssq = 0.f;
  const u16* xr = a.x + (xrow ? r : 0) * a.ldx + 8 * kq;
  const u16* wr[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
    wr[j] = a.seg[MODE == 2 ? j : s].w + (int64_t)min(n0 + r, sg.n - 1) * K + 8 * kq;

  f32x4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // MODE 1: the residual values of this lane's outputs (rows m = 4 kq + e, column n0 + r), loaded at
  // entry so their latency overlaps the weight stream instead of following the fold
  [[maybe_unused]] u16 resv[4];
  if constexpr (MODE == 1) {
    const int nr = min(n0 + r, sg.n - 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) resv[e] = a.res[(int64_t)min(4 * kq + e, M - 1) * a.ldres + nr];
  }

  // Q blocks of 128 k at kb[0..Q): all loads first, then the MFMAs.  `guard` bounds each 16-byte
  // chunk by K (the ragged last block).
  auto blocks = [&](auto qc, const int* kb, bool guard) {
    constexpr int Q = decltype(qc)::value;
    i32x4 wv[Q][NB][4], xv[Q][4], nv[Q][4];
#pragma unroll
    for (int p = 0; p < Q; ++p)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = kb[p] + 32 * c + 8 * kq;
        const bool ok = !guard || k < K;
#pragma unroll
        for (int j = 0; j < NB; ++j)
          wv[p][j][c] = ok ? *reinterpret_cast<const i32x4*>(wr[j] + kb[p] + 32 * c) : i32x4{0, 0, 0, 0};
        xv[p][c] = ok && xrow ? *reinterpret_cast<const i32x4*>(xr + kb[p] + 32 * c) : i32x4{0, 0, 0, 0};
        if constexpr (NORM) nv[p][c] = ok ? *reinterpret_cast<const i32x4*>(a.nw + k) : i32x4{0, 0, 0, 0};
      }
#pragma unroll
    for (int p = 0; p < Q; ++p)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        i32x4 xf = xv[p][c];
        if constexpr (NORM) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t xx = (uint32_t)xv[p][c][w], ww = (uint32_t)nv[p][c][w];
            const float x0 = to_f32<T>((u16)(xx & 0xffffu)), x1 = to_f32<T>((u16)(xx >> 16));
            ssq += x0 * x0 + x1 * x1;
            xf[w] = (int)pack2<T>(x0 * to_f32<T>((u16)(ww & 0xffffu)), x1 * to_f32<T>((u16)(ww >> 16)));
          }
        }
#pragma unroll
        for (int j = 0; j < NB; ++j)
          acc[j] = mfma_16x16x32<T>(__builtin_bit_cast(bf16x8_t, xf), __builtin_bit_cast(bf16x8_t, wv[p][j][c]), acc[j]);
      }
  };
  const int nfull = K / 128, nblk = (K + 127) / 128;
  int b = wave;
  for (; b + (P - 1) * NW < nfull; b += P * NW) {  // P blocks in flight per wave
    int kb[P];
#pragma unroll
    for (int p = 0; p < P; ++p) kb[p] = (b + p * NW) * 128;
    blocks(std::integral_constant<int, P>{}, kb, false);
  }
  for (; b < nblk; b += NW) {
    const int kb[1] = {b * 128};
    blocks(std::integral_constant<int, 1>{}, kb, b >= nfull);
  }

#pragma unroll
  for (int j = 0; j < NB; ++j) red[wave][j][lane] = acc[j];
  if constexpr (NORM) red_ss[wave][lane] = ssq;
  __syncthreads();
  if (wave != 0) return;
  float v[NB][4];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    f32x4 t = red[0][j][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[w][j][lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[j][e] = t[e];
  }
  if constexpr (NORM) {
    // lane (r, kq) holds row r's squares over its k chunks: fold the waves, then the 4 quarters
    float t = red_ss[0][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red_ss[w][lane];
    t += __shfl_xor(t, 16, 64);
    t += __shfl_xor(t, 32, 64);
    const float inv_r = rsqrtf(t * (1.f / (float)K) + a.eps);  // row r's scale
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float inv_m = __shfl(inv_r, 4 * kq + e, 64);       // the scale of output row m = 4 kq + e
#pragma unroll
      for (int j = 0; j < NB; ++j) v[j][e] *= inv_m;
    }
  }
  // lane holds D[m = 4 kq + e][n = r]
  const int n = n0 + r;
  if (n >= sg.n) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = 4 * kq + e;
    if (m >= M) continue;
    float o = to_f32<T>(from_f32<T>(v[0][e]));
    if constexpr (MODE == 1) o = to_f32<T>(resv[e]) + o;
    if constexpr (MODE == 2) {
      const float u = to_f32<T>(from_f32<T>(v[1][e]));
      o = o * q3_sigmoid(o) * u;
    }
    sg.y[m * sg.ldy + n] = from_f32<T>(o);
  }
}

// Persistent variant for K = NW * KB * 128 (Qwen3-8B: K = 4096) and modes 0 / 2: the input rows (the
// RMSNorm-weighted rows when NORM) are read once per workgroup and stay in registers, and "units" of
// 16 weight rows (mode 2: a gate unit, then the up unit of the same rows) stream through a two-deep
// register pipeline -- the loads of the next unit are in flight while the current unit's MFMAs and
// its cross-wave fold run.  The sum of squares of the input rows is formed once per workgroup, while
// the first unit's weights are already in flight.  Lane (r, kq) of wave w holds k = (w + NW i) * 128
// + 32 c + 8 kq, i < KB, c < 4, of token row r (A operand) and weight row n0 + r (B operand); the
// waves' partial 16 x 16 tiles fold in LDS in wave order (fixed order: deterministic).
// RU = 8 (mode 0, at most 8 token rows): units of 8 weight rows, so that a launch whose 16-row units
// would leave CUs idle (Q/K/V: 384 units of 16 rows on 256 CUs) divides evenly (768 units of 8).  Each
// 64-wide k step is split in two 32-wide halves h that sit on different MFMA rows and columns: lane
// (r, kq) takes weight row r % 8 and token row r % 8 at k = 64 c + 32 h + 8 kq with h = r / 8, so
// D[m + 8 h][n + 8 h] is half h of the dot product of token row m and weight row n (the cross-half
// blocks are unused), and every load instruction reads 128 contiguous bytes of 8 rows.
template <typename T, int MODE, bool NORM, int NW, int KB, int RU = 16>
__global__ __launch_bounds__(NW * 64) void dlinear_stream_kernel(DecArgs a, int units) {
  static_assert(MODE == 0 || MODE == 2, "projection or SwiGLU");
  static_assert(RU == 16 || (RU == 8 && MODE == 0), "8-row units: projections only");
  constexpr int CPB = RU == 16 ? 4 : 2;  // 16-byte chunks per lane and 128-wide k block
  __shared__ f32x4 red[2][NW][64];
  __shared__ float red_ss[NW][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, kq = lane >> 4;
  const int rr = RU == 16 ? r : (r & 7), hh = RU == 16 ? 0 : (r >> 3);  // unit row, k half (RU 8)
  const int M = a.M, K = a.K;
  const bool xrow = rr < M;
  auto koff = [&](int i, int c) {
    return (wave + NW * i) * 128 + (RU == 16 ? 32 * c + 8 * kq : 64 * c + 32 * hh + 8 * kq);
  };
  auto unit_src = [&](int u, const u16*& w, int& n0, int& nrows) {
    if constexpr (MODE == 2) {
      w = a.seg[u & 1].w;
      n0 = (u >> 1) * 16;
      nrows = a.seg[0].n;
    } else {
      int s = 0, t = u;
      while (s + 1 < a.nseg && t >= a.seg[s].tiles) t -= a.seg[s++].tiles;
      w = a.seg[s].w;
      n0 = t * RU;
      nrows = a.seg[s].n;
    }
  };
  constexpr int LPU = KB * CPB;  // weight loads per unit and lane
  i32x4 xv[KB][CPB];
  float inv_m[4] = {1.f, 1.f, 1.f, 1.f};
  i32x4 wb[2][KB][CPB];
  auto issue = [&](int u, auto buf_c) {
    constexpr int B = decltype(buf_c)::value;
    const u16* w;
    int n0, nrows;
    unit_src(u, w, n0, nrows);
    const u16* row = w + (int64_t)min(n0 + rr, nrows - 1) * K;
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
      for (int c = 0; c < CPB; ++c) wb[B][i][c] = *reinterpret_cast<const i32x4*>(row + koff(i, c));
  };
  float gate[4] = {0.f, 0.f, 0.f, 0.f};
  // wave 0: fold the waves' partial tiles in order, then the epilogue (lane holds D[m = 4 kq + e][n = r])
  auto finish = [&](int u, int par) {
    f32x4 t = red[par][0][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[par][w][lane];
    if constexpr (RU == 8) {
      // D[m][n] (lane n + 16 (m / 4), n < 8, m < 8) + D[m + 8][n + 8] (that lane + 40)
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] += __shfl(t[e], (lane + 40) & 63, 64);
    }
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = t[e] * inv_m[e];
    if constexpr (MODE == 2) {
      if ((u & 1) == 0) {  // gate unit: kept for the up unit that follows
#pragma unroll
        for (int e = 0; e < 4; ++e) gate[e] = v[e];
        return;
      }
    }
    int s = 0, tt = u;
    if constexpr (MODE == 2) {
      tt = u >> 1;
    } else {
      while (s + 1 < a.nseg && tt >= a.seg[s].tiles) tt -= a.seg[s++].tiles;
    }
    const DecSeg sg = a.seg[s];
    if (RU == 8 && (r >= 8 || kq >= 2)) return;
    const int n = tt * RU + r;
    if (n >= sg.n) return;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 4 * kq + e;
      if (m >= M) continue;
      float o = to_f32<T>(from_f32<T>(v[e]));
      if constexpr (MODE == 2) {
        const float g = to_f32<T>(from_f32<T>(gate[e]));
        o = g * q3_sigmoid(g) * o;
      }
      sg.y[m * sg.ldy + n] = from_f32<T>(o);
    }
  };
  auto compute = [&](auto buf_c) {
    constexpr int B = decltype(buf_c)::value;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
      for (int c = 0; c < CPB; ++c)
        acc = mfma_16x16x32<T>(__builtin_bit_cast(bf16x8_t, xv[i][c]), __builtin_bit_cast(bf16x8_t, wb[B][i][c]), acc);
    return acc;
  };
  // this workgroup's units: blockIdx.x, + gridDim.x, ... (mode 2: the (gate, up) unit pairs of those tiles)
  const int step = MODE == 2 ? 2 * gridDim.x : gridDim.x;
  int u = MODE == 2 ? 2 * blockIdx.x : blockIdx.x;
  auto next_u = [&](int v) { return MODE == 2 ? ((v & 1) ? v - 1 + step : v + 1) : v + step; };
  if (u >= units) return;  // uniform over the workgroup
  i32x4 nvv[NORM ? KB : 1][CPB];
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int c = 0; c < CPB; ++c) {
      const int k = koff(i, c);
      xv[i][c] = *reinterpret_cast<const i32x4*>(a.x + (int64_t)(xrow ? rr : 0) * a.ldx + k);
      if constexpr (NORM) nvv[i][c] = *reinterpret_cast<const i32x4*>(a.nw + k);
    }
  issue(u, std::integral_constant<int, 0>{});
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int c = 0; c < CPB; ++c)
      if (!xrow) xv[i][c] = i32x4{0, 0, 0, 0};
  if constexpr (NORM) {
    // the input rows and norm weight landed (older than the first unit's weight loads)
    __builtin_amdgcn_s_waitcnt((LPU & 15) | ((LPU >> 4) << 14) | (7 << 4) | (0xF << 8));
    float ssq = 0.f;
#pragma unroll
    for (int i = 0; i < KB; ++i)
#pragma unroll
      for (int c = 0; c < CPB; ++c)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t xx = (uint32_t)xv[i][c][w], ww = (uint32_t)nvv[i][c][w];
          const float x0 = to_f32<T>((u16)(xx & 0xffffu)), x1 = to_f32<T>((u16)(xx >> 16));
          ssq += x0 * x0 + x1 * x1;
          xv[i][c][w] = (int)pack2<T>(x0 * to_f32<T>((u16)(ww & 0xffffu)), x1 * to_f32<T>((u16)(ww >> 16)));
        }
    ssq += __shfl_xor(ssq, 16, 64);  // row r over the 4 quarters (RU 8: and both k halves), then over the waves
    ssq += __shfl_xor(ssq, 32, 64);
    if constexpr (RU == 8) ssq += __shfl_xor(ssq, 8, 64);
    red_ss[wave][lane] = ssq;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += red_ss[w][lane];
    const float inv_r = rsqrtf(t * (1.f / (float)K) + a.eps);
#pragma unroll
    for (int e = 0; e < 4; ++e) inv_m[e] = __shfl(inv_r, 4 * kq + e, 64);
  }
  // Two units per trip (register buffers 0 and 1); the LDS fold buffer alternates with the unit, so one
  // barrier per unit suffices (wave 0 has read a buffer before any wave passes the next barrier).
  int it = 0;
  auto one = [&](auto cur_c, int cu, bool more) {
    constexpr int CUR = decltype(cur_c)::value;
    __builtin_amdgcn_sched_barrier(0);
    if (more) issue(next_u(cu), std::integral_constant<int, CUR ^ 1>{});
    __builtin_amdgcn_sched_barrier(0);
    if (more) __builtin_amdgcn_s_waitcnt((LPU & 15) | ((LPU >> 4) << 14) | (7 << 4) | (0xF << 8));
    else __builtin_amdgcn_s_waitcnt((7 << 4) | (0xF << 8));
    red[it & 1][wave][lane] = compute(cur_c);
    __syncthreads();
    if (wave == 0) finish(cu, it & 1);
    ++it;
  };
  while (true) {
    const int u1 = next_u(u);
    one(std::integral_constant<int, 0>{}, u, u1 < units);
    if (u1 >= units) break;
    const int u2 = next_u(u1);
    one(std::integral_constant<int, 1>{}, u1, u2 < units);
    if (u2 >= units) break;
    u = u2;
  }
}

// Waves per workgroup x k blocks in flight per wave, per mode: measured on MI355X over {4, 8, 16} waves
// x {1, 2, 4} blocks, each projection kind separately (36 distinct weights per captured graph): modes
// 0 / 2 (shapes the streaming kernel does not take) 8 x 2 and 8 x 1; mode 1 (O and down + residual)
// 8 x 4 up to K = 4096 (every block of a wave in flight: O 9.0 -> 8.2 us at B1), 8 x 1 above (down,
// K = 12288: more blocks in flight measured slower at B8).
template <typename T, int MODE, bool NORM>
int dlinear_launch(const DecArgs& a, int tiles, hipStream_t s) {
  constexpr int NW = 8;
  if constexpr (MODE == 1) {
    if (a.K <= 4096) {
      dlinear_kernel<T, MODE, NORM, NW, 4><<<(unsigned)tiles, NW * 64, 0, s>>>(a);
      return (int)hipGetLastError();
    }
  }
  dlinear_kernel<T, MODE, NORM, NW, MODE == 0 ? 2 : 1><<<(unsigned)tiles, NW * 64, 0, s>>>(a);
  return (int)hipGetLastError();
}

// Units per workgroup of the streaming kernel, by the number of 16-row tiles (pairs in mode 2); measured
// inside a captured 36-layer step on MI355X: 2 for Q/K/V (384 tiles), 3 for gate/up (768 pairs); one
// unit per workgroup up to 256 tiles; above 1024 (the LM head, 9496 tiles) one round of 256 workgroups
// (B1 3.339 -> 3.323 ms per token against 8 units per workgroup on 1187 workgroups).
inline int stream_units_per_wg(int tiles) { return tiles <= 256 ? 1 : tiles <= 512 ? 2 : tiles <= 1024 ? 3 : (tiles + 255) / 256; }

template <typename T, int MODE, bool NORM, int KB>
int dlinear_stream_launch(const DecArgs& a, int tiles, hipStream_t s) {
  const int upw = stream_units_per_wg(tiles);
  const int units = MODE == 2 ? 2 * tiles : tiles;
  dlinear_stream_kernel<T, MODE, NORM, 8, KB><<<(unsigned)((tiles + upw - 1) / upw), 512, 0, s>>>(a, units);
  return (int)hipGetLastError();
}

// 8-row units for a projection of at most 8 token rows whose 16-row units would need two per
// workgroup on fewer workgroups than CUs (256 < tiles <= 512).
template <typename T, bool NORM, int KB>
int dlinear_stream_r8(const DecArgs& a0, hipStream_t s) {
  DecArgs a = a0;
  int units = 0;
  for (int i = 0; i < a.nseg; ++i) units += (a.seg[i].tiles = (a.seg[i].n + 7) / 8);
  const int upw = stream_units_per_wg(units);
  dlinear_stream_kernel<T, 0, NORM, 8, KB, 8><<<(unsigned)((units + upw - 1) / upw), 512, 0, s>>>(a, units);
  return (int)hipGetLastError();
}

template <typename T, int MODE, bool NORM>
int dlinear_stream_k(const DecArgs& a, int tiles, hipStream_t s) {
  if constexpr (MODE == 0) {
    if (a.M <= 8 && tiles > 256 && tiles <= 512) {
      if (a.K == 1024) return dlinear_stream_r8<T, NORM, 1>(a, s);
      if (a.K == 2048) return dlinear_stream_r8<T, NORM, 2>(a, s);
      return dlinear_stream_r8<T, NORM, 4>(a, s);
    }
  }
  if (a.K == 1024) return dlinear_stream_launch<T, MODE, NORM, 1>(a, tiles, s);
  if (a.K == 2048) return dlinear_stream_launch<T, MODE, NORM, 2>(a, tiles, s);
  return dlinear_stream_launch<T, MODE, NORM, 4>(a, tiles, s);
}

template <typename T>
int dlinear_t(const DecArgs& a, int tiles, int mode, bool norm, hipStream_t s) {
  if ((a.K == 1024 || a.K == 2048 || a.K == 4096) && mode != 1 && a.ldx % 8 == 0) {
    if (mode == 0) return norm ? dlinear_stream_k<T, 0, true>(a, tiles, s) : dlinear_stream_k<T, 0, false>(a, tiles, s);
    return norm ? dlinear_stream_k<T, 2, true>(a, tiles, s) : dlinear_stream_k<T, 2, false>(a, tiles, s);
  }
  if (mode == 0) return norm ? dlinear_launch<T, 0, true>(a, tiles, s) : dlinear_launch<T, 0, false>(a, tiles, s);
  if (mode == 1) return norm ? dlinear_launch<T, 1, true>(a, tiles, s) : dlinear_launch<T, 1, false>(a, tiles, s);
  return norm ? dlinear_launch<T, 2, true>(a, tiles, s) : dlinear_launch<T, 2, false>(a, tiles, s);
}

// ============================================================================ KV append
// cache[b, h, start + s, :] = kv[b, s, h, :] for K and V ([B,S,H,D] -> [B,H,C,D]), 16-byte moves.
// With start_dev the position is read from device memory (graph-replayable decode steps);
// positions at or beyond the capacity are never written.
__global__ __launch_bounds__(kThreads) void kv_append_kernel(const u16* __restrict__ k, const u16* __restrict__ v,
                                                             u16* __restrict__ ck, u16* __restrict__ cv, int S, int H,
                                                             int D, int C, int start, const int64_t* start_dev,
                                                             int64_t nvec) {
  if (start_dev) start = (int)*start_dev;
  const int dv = D / 8;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < nvec; i += stride) {
    const int c = (int)(i % dv);
    const int64_t rest = i / dv;
    const int h = (int)(rest % H), s = (int)((rest / H) % S);
    const int64_t b = rest / ((int64_t)H * S);
    if (start + s >= C || start < 0) continue;
    const int64_t dst = (((b * H + h) * C) + start + s) * D + c * 8;
    const int64_t src = rest * D + c * 8;
    *reinterpret_cast<i32x4*>(ck + dst) = *reinterpret_cast<const i32x4*>(k + src);
    *reinterpret_cast<i32x4*>(cv + dst) = *reinterpret_cast<const i32x4*>(v + src);
  }
}

// ============================================================================ decode attention
// One workgroup (NWV waves) per (b, kv head, split of 16 NWV cached keys) computes all G
// query heads of the GQA group, so every K/V byte is read once; each wave owns 16 keys and issues all
// of its K and V loads before using any.  A second kernel merges the splits in fixed order
// (deterministic).

struct DecAttnArgs {
  const u16* q;  // [B, Hq, D] at strides (qsb, qsh)
  int64_t qsb, qsh;
  u16* ck;
  u16* cv;  // caches [.., capacity, D] at strides (ksb, ksh)
  int64_t ksb, ksh;
  float* opart;
  float* mpart;
  float* lpart;
  int Hkv, T_len, capacity, splits;
  const int64_t* len_dev;
  float scale2;
  // FUSED: q and the new token's k, v are raw projections; QK-norm + RoPE and the cache append
  // happen here.
  const u16* k;
  const u16* v;  // [B, Hkv, D] at strides (kvsb, kvsh)
  int64_t kvsb, kvsh;
  const u16* qw;
  const u16* kw;
  float eps;
  const u16* cs;
  const u16* sn;  // [B, D] rotary tables of the token's position, batch stride csb
  int64_t csb;
};

// Per wave:
// S^T = K q^T on v_mfma_f32_16x16x32 (K rows loaded straight into the A-operand layout, the group's
// G query rows -- normalised once per workgroup, one wave per head -- as the B operand padded to 16
// columns); the accumulator layout of S^T (lane: head l % 16, keys 4 (l / 16) .. + 3) is exactly the
// A-operand layout of P for O = P V on v_mfma_f32_16x16x16, whose V operand (4 consecutive keys of
// one dimension per lane) comes from the wave's V tile in LDS through the gfx950 transpose read.
// The softmax max and sum are formed per head over the workgroup's 16 NWV keys (lane butterflies,
// then the waves through LDS); P is rounded to the storage type for the P V product, as in the
// prefill kernels.
typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
template <typename T> Q3_DEV f32x4 mfma_16x16x16(i32x2 a, i32x2 b, f32x4 c);
template <> Q3_DEV f32x4 mfma_16x16x16<BF16>(i32x2 a, i32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4s_t, a), __builtin_bit_cast(v4s_t, b), c, 0, 0,
                                                   0);
}
template <> Q3_DEV f32x4 mfma_16x16x16<F16>(i32x2 a, i32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h_t, a), __builtin_bit_cast(v4h_t, b), c, 0, 0, 0);
}

// RMSNorm + rotate-half RoPE of one 128-dim row held 2 dims per lane (lane l: dims 2 l, 2 l + 1; the
// partner dims 64 away live in lane l ^ 32), rounded to the storage type exactly like the standalone
// QK-norm + RoPE kernel.
template <typename T>
Q3_DEV void norm_rope2(float& x0, float& x1, uint32_t w, uint32_t cs, uint32_t sn, int lane, float eps) {
  const float inv = rsqrtf(group_sum<64>(x0 * x0 + x1 * x1) * (1.f / 128.f) + eps);
  const float n0 = x0 * inv * to_f32<T>((u16)(w & 0xffffu)), n1 = x1 * inv * to_f32<T>((u16)(w >> 16));
  const float p0 = __shfl_xor(n0, 32, 64), p1 = __shfl_xor(n1, 32, 64);
  const float sign = lane < 32 ? -1.f : 1.f;
  x0 = to_f32<T>(from_f32<T>(n0 * to_f32<T>((u16)(cs & 0xffffu)) + sign * p0 * to_f32<T>((u16)(sn & 0xffffu))));
  x1 = to_f32<T>(from_f32<T>(n1 * to_f32<T>((u16)(cs >> 16)) + sign * p1 * to_f32<T>((u16)(sn >> 16))));
}

template <typename T, int G, bool FUSED, int NWV>
__global__ __launch_bounds__(NWV * 64) void decode_attn_mfma_kernel(DecAttnArgs a) {
  constexpr int D = 128, KPW = 16, HPW = (G + NWV - 1) / NWV;  // keys and query heads per wave
  constexpr int kSplit = KPW * NWV;
  __shared__ __attribute__((aligned(16))) u16 vt[NWV][KPW * D];  // per-wave V tile, 16-byte chunks swizzled
  __shared__ __attribute__((aligned(16))) u16 qs[G][D];
  __shared__ __attribute__((aligned(16))) u16 knew[D];
  __shared__ float wred[2][NWV][16];
  __shared__ float red_o[NWV][G][D];
  const int split = blockIdx.x, bk = blockIdx.y, b = bk / a.Hkv, hk = bk % a.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int k0 = split * kSplit, kw = k0 + wave * KPW;
  u16* kb = a.ck + b * a.ksb + hk * a.ksh;
  u16* vb = a.cv + b * a.ksb + hk * a.ksh;
  // Every global load first (cache rows read unconditionally up to the capacity, masked below):
  // K A-operand fragments (lane (r, kq): key kw + r, dims 32 s + 8 kq), V rows (lane: key kw + lane / 4,
  // 16-byte chunks lane % 4 + 4 c), this wave's query rows and the new token's k / v with the tables.
  i32x4 kf[4], vr[4];
  const int64_t krow = (int64_t)min(kw + r, a.capacity - 1) * D;
#pragma unroll
  for (int s = 0; s < 4; ++s) kf[s] = *reinterpret_cast<const i32x4*>(kb + krow + 32 * s + 8 * kq);
  const int vkey = lane >> 2;
  const int64_t vrow = (int64_t)min(kw + vkey, a.capacity - 1) * D;
#pragma unroll
  for (int c = 0; c < 4; ++c) vr[c] = *reinterpret_cast<const i32x4*>(vb + vrow + ((lane & 3) + 4 * c) * 8);
  uint32_t qraw[HPW];
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    const int h = min(wave + NWV * i, G - 1);
    qraw[i] = *reinterpret_cast<const uint32_t*>(a.q + b * a.qsb + (int64_t)(hk * G + h) * a.qsh + 2 * lane);
  }
  uint32_t kraw = 0u, vraw = 0u, qwv = 0u, kwv = 0u, csv = 0u, snv = 0u;
  i32x4 vnew[4] = {};
  if constexpr (FUSED) {
    const u16* kn = a.k + b * a.kvsb + hk * a.kvsh;
    const u16* vn = a.v + b * a.kvsb + hk * a.kvsh;
    kraw = *reinterpret_cast<const uint32_t*>(kn + 2 * lane);
    vraw = *reinterpret_cast<const uint32_t*>(vn + 2 * lane);
#pragma unroll
    for (int c = 0; c < 4; ++c) vnew[c] = *reinterpret_cast<const i32x4*>(vn + ((lane & 3) + 4 * c) * 8);
    qwv = *reinterpret_cast<const uint32_t*>(a.qw + 2 * lane);
    kwv = *reinterpret_cast<const uint32_t*>(a.kw + 2 * lane);
    csv = *reinterpret_cast<const uint32_t*>(a.cs + b * a.csb + 2 * lane);
    snv = *reinterpret_cast<const uint32_t*>(a.sn + b * a.csb + 2 * lane);
  }
  // len_dev holds the cache length before this token: the token itself is at that position.
  const int pos = a.len_dev ? (int)*a.len_dev : a.T_len - 1;
  const int T_len = a.len_dev ? min(pos + 1, a.capacity) : a.T_len;
  const bool own = FUSED && pos >= k0 && pos < k0 + kSplit && pos < a.capacity;  // this split holds the token

  // query rows of this wave's heads (normalised + rotated when fused) -> LDS
#pragma unroll
  for (int i = 0; i < HPW; ++i) {
    const int h = wave + NWV * i;
    if (h < G) {
      float x0 = to_f32<T>((u16)(qraw[i] & 0xffffu)), x1 = to_f32<T>((u16)(qraw[i] >> 16));
      if constexpr (FUSED) norm_rope2<T>(x0, x1, qwv, csv, snv, lane, a.eps);
      *reinterpret_cast<uint32_t*>(&qs[h][2 * lane]) = pack2<T>(x0, x1);
    }
  }
  if constexpr (FUSED) {
    if (own && wave == 0) {  // the new token: k = rope(norm(k_raw)), v raw; into the cache and into LDS
      float x0 = to_f32<T>((u16)(kraw & 0xffffu)), x1 = to_f32<T>((u16)(kraw >> 16));
      norm_rope2<T>(x0, x1, kwv, csv, snv, lane, a.eps);
      const uint32_t kp = pack2<T>(x0, x1);
      *reinterpret_cast<uint32_t*>(&knew[2 * lane]) = kp;
      *reinterpret_cast<uint32_t*>(kb + (int64_t)pos * D + 2 * lane) = kp;
      *reinterpret_cast<uint32_t*>(vb + (int64_t)pos * D + 2 * lane) = vraw;
    }
  }
  // V tile: rows past the length zeroed (their probabilities are 0, but the cache may hold anything),
  // the new token's row from its raw v
  {
    const bool live = kw + vkey < T_len;
    const bool mine = own && kw + vkey == pos;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      i32x4 val = mine ? vnew[c] : live ? vr[c] : i32x4{0, 0, 0, 0};
      const int ch = ((lane & 3) + 4 * c) ^ (2 * (vkey & 7));
      *reinterpret_cast<i32x4*>(&vt[wave][vkey * D + ch * 8]) = val;
    }
  }
  __syncthreads();
  if (own && pos >= kw && pos < kw + KPW && r == pos - kw) {  // the new key's fragments
#pragma unroll
    for (int s = 0; s < 4; ++s) kf[s] = *reinterpret_cast<const i32x4*>(&knew[32 * s + 8 * kq]);
  }
  // S^T = K q^T (16 keys x 16 heads, heads >= G are zero columns)
  f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const i32x4 qf = r < G ? *reinterpret_cast<const i32x4*>(&qs[min(r, G - 1)][32 * s + 8 * kq]) : i32x4{0, 0, 0, 0};
    sacc = mfma_16x16x32<T>(__builtin_bit_cast(bf16x8_t, kf[s]), __builtin_bit_cast(bf16x8_t, qf), sacc);
  }
  float sv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) sv[e] = (kw + 4 * kq + e < T_len && r < G) ? sacc[e] * a.scale2 : -INFINITY;
  float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (kq == 0) wred[0][wave][r] = mx;
  __syncthreads();
  float m = wred[0][0][r];
#pragma unroll
  for (int w = 1; w < NWV; ++w) m = fmaxf(m, wred[0][w][r]);
  float p[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) p[e] = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[e] - m);
  float sum = (p[0] + p[1]) + (p[2] + p[3]);
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  if (kq == 0) wred[1][wave][r] = sum;
  // O = P V over this wave's 16 keys, 8 blocks of 16 dims
  const i32x2 pa = i32x2{(int)pack2<T>(p[0], p[1]), (int)pack2<T>(p[2], p[3])};
  const int trow = 4 * kq + (r >> 2);
  const char* vbase = reinterpret_cast<const char*>(&vt[wave][trow * D]);
  f32x4 o[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    const int cb = 32 * db + 8 * (r & 3);  // byte offset of the 4 dims this lane addresses
    const char* pv = vbase + ((((cb >> 4) ^ (2 * (trow & 7)))) << 4) + (cb & 15);
    const i32x2 vf = __builtin_bit_cast(
        i32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)pv));
    o[db] = mfma_16x16x16<T>(pa, vf, f32x4{0.f, 0.f, 0.f, 0.f});
  }
  // o[db][e] = O[head 4 kq + e][dim 16 db + r]
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (4 * kq + e < G) red_o[wave][4 * kq + e][16 * db + r] = o[db][e];
  __syncthreads();
  const int64_t pbase = ((int64_t)bk * a.splits + split) * G;
  for (int i = tid; i < G * D; i += NWV * 64) {
    const int g = i / D, d = i % D;
    float o = red_o[0][g][d];
#pragma unroll
    for (int w = 1; w < NWV; ++w) o += red_o[w][g][d];
    a.opart[(pbase + g) * D + d] = o;
  }
  if (tid < G) {
    float mx2 = wred[0][0][tid], l = wred[1][0][tid];
#pragma unroll
    for (int w = 1; w < NWV; ++w) {
      mx2 = fmaxf(mx2, wred[0][w][tid]);
      l += wred[1][w][tid];
    }
    a.mpart[pbase + tid] = mx2;
    a.lpart[pbase + tid] = l;
  }
}

// out[b, hq, :] = sum_j exp2(m_j - M) o_j / sum_j exp2(m_j - M) l_j over the splits, in fixed order.
// One workgroup of 4 x 128 threads per (b, query head): the split weights go to LDS once, thread
// group r sums the splits j = r mod 4 with all its loads in flight, and the 4 groups fold in LDS.
template <typename T, int G>
__global__ __launch_bounds__(512) void decode_merge_kernel(const float* __restrict__ opart,
                                                           const float* __restrict__ mpart,
                                                           const float* __restrict__ lpart, u16* __restrict__ out,
                                                           int64_t osb, int64_t osh, int Hq, int splits) {
  constexpr int D = 128, MAXS = 1024;
  __shared__ float wgt[MAXS];
  __shared__ float part[4][D];
  __shared__ float red[16];
  const int bh = blockIdx.x, b = bh / Hq, h = bh % Hq, bk = bh / G, g = bh % G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = tid >> 7, d = tid & 127;
  // First iterations' loads up front (clamped indices, masked where used), so one memory latency
  // covers the max, the weights and the first block of partial outputs.
  const int64_t p0 = ((int64_t)bk * splits + min(tid, splits - 1)) * G + g;
  const float m0 = mpart[p0], l0 = lpart[p0];
  float x0[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) x0[u] = opart[(((int64_t)bk * splits + min(r + 4 * u, splits - 1)) * G + g) * D + d];
  // global max and denominator over the splits (the whole workgroup, fixed reduction order)
  float mx = tid < splits ? m0 : -INFINITY;
  for (int j = tid + 512; j < splits; j += 512) mx = fmaxf(mx, mpart[((int64_t)bk * splits + j) * G + g]);
  mx = group_max<64>(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < 8; ++w) M = fmaxf(M, red[w]);
  float den = 0.f;
  for (int j = tid; j < splits; j += 512) {
    const int64_t pj = ((int64_t)bk * splits + j) * G + g;
    const float mj = j == tid ? m0 : mpart[pj];
    const float w = mj == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mj - M);  // split with no live key
    wgt[j] = w;
    den += w * (j == tid ? l0 : lpart[pj]);
  }
  den = group_sum<64>(den);
  __syncthreads();  // red[] reads done; wgt[] complete
  if (lane == 0) red[8 + wave] = den;
  float acc = 0.f;
  for (int j0 = r; j0 < splits; j0 += 4 * 8) {
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + 4 * u;
      x[u] = j0 == r ? x0[u] : j < splits ? opart[(((int64_t)bk * splits + j) * G + g) * D + d] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + 4 * u;
      if (j < splits) acc += wgt[j] * x[u];
    }
  }
  part[r][d] = acc;
  __syncthreads();
  if (tid < D) {
    float tot = red[8];
#pragma unroll
    for (int w = 1; w < 8; ++w) tot += red[8 + w];
    const float y = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
    out[b * osb + (int64_t)h * osh + tid] = from_f32<T>(y / tot);
  }
}

// ============================================================================ greedy select
// Stage 1: each workgroup reduces a slice of one row to (max, lowest index of the max).
template <typename T>
__global__ __launch_bounds__(kThreads) void argmax_parts_kernel(const typename T::storage* __restrict__ x,
                                                                int64_t ldx, int64_t n, float* __restrict__ pv,
                                                                int* __restrict__ pi, int parts) {
  __shared__ float sv[kThreads];
  __shared__ int si[kThreads];
  const int row = blockIdx.y, part = blockIdx.x;
  const int64_t per = (n + parts - 1) / parts;
  const int64_t lo = (int64_t)part * per, hi = min(n, lo + per);
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) {
    const float v = to_f32<T>(x[row * ldx + i]);
    if (v > best) {  // increasing i per thread: the first max seen is the lowest index
      best = v;
      bi = (int)i;
    }
  }
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int o = kThreads / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      const float v2 = sv[threadIdx.x + o];
      const int i2 = si[threadIdx.x + o];
      if (v2 > sv[threadIdx.x] || (v2 == sv[threadIdx.x] && i2 < si[threadIdx.x])) {
        sv[threadIdx.x] = v2;
        si[threadIdx.x] = i2;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pv[row * parts + part] = sv[0];
    pi[row * parts + part] = si[0];
  }
}

// Stage 2 (one thread per row): token = argmax (lowest index on ties); rows already done emit pad;
// ids[row, pos] = next[row] = token; done |= token in eos.
__global__ void select_kernel(const float* __restrict__ pv, const int* __restrict__ pi, int parts,
                              int64_t* __restrict__ ids, int64_t ld_ids, int64_t pos, const int64_t* pos_dev,
                              int64_t* __restrict__ next, uint8_t* __restrict__ done,
                              const int64_t* __restrict__ eos, int n_eos, int64_t pad, int batch) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= batch) return;
  if (pos_dev) pos += *pos_dev;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int j = 0; j < parts; ++j) {
    const float v = pv[row * parts + j];
    const int i = pi[row * parts + j];
    if (v > best || (v == best && i < bi)) {
      best = v;
      bi = i;
    }
  }
  const bool was_done = done[row] != 0;
  const int64_t tok = was_done ? pad : (int64_t)bi;
  bool end = false;
  for (int e = 0; e < n_eos; ++e) end = end || (tok == eos[e]);
  if (ids && pos >= 0 && pos < ld_ids) ids[row * ld_ids + pos] = tok;
  next[row] = tok;
  done[row] = (was_done || end) ? 1 : 0;
}

// *counter += by (single thread): advances a device-resident cache length between replays.
__global__ void advance_kernel(int64_t* counter, int64_t by) { *counter += by; }

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Keys per split: 128 (8 waves of 16 keys).  Measured in the captured 36-layer step (2048 + 128-token
// B1, 1024 + 128-token B8): 64-key splits 3.376 / 3.851 ms, 128: 3.346 / 3.836, 256: 3.444 / 4.049.
constexpr int kSplitWaves = 8, kSplitKeys = 16 * kSplitWaves;
// Workspace: per (b, kv head, split, head of the group) 128 partial outputs, then the maxima, then
// the sums.
int64_t decode_splits(int64_t span) { return (span + kSplitKeys - 1) / kSplitKeys; }

template <typename T, int G, bool FUSED>
int decode_g(const DecAttnArgs& a, dim3 grid, void* out, int64_t osb, int64_t osh, hipStream_t s) {
  decode_attn_mfma_kernel<T, G, FUSED, kSplitWaves><<<grid, kSplitWaves * 64, 0, s>>>(a);
  decode_merge_kernel<T, G><<<grid.y * G, 512, 0, s>>>(a.opart, a.mpart, a.lpart, (u16*)out, osb, osh, a.Hkv * G,
                                                       a.splits);
  return (int)hipGetLastError();
}

template <typename T, bool FUSED>
int decode_t(int G, const DecAttnArgs& a, dim3 grid, void* out, int64_t osb, int64_t osh, hipStream_t s) {
  switch (G) {
    case 1: return decode_g<T, 1, FUSED>(a, grid, out, osb, osh, s);
    case 2: return decode_g<T, 2, FUSED>(a, grid, out, osb, osh, s);
    case 3: return decode_g<T, 3, FUSED>(a, grid, out, osb, osh, s);
    case 4: return decode_g<T, 4, FUSED>(a, grid, out, osb, osh, s);
    case 5: return decode_g<T, 5, FUSED>(a, grid, out, osb, osh, s);
    case 6: return decode_g<T, 6, FUSED>(a, grid, out, osb, osh, s);
    case 7: return decode_g<T, 7, FUSED>(a, grid, out, osb, osh, s);
    case 8: return decode_g<T, 8, FUSED>(a, grid, out, osb, osh, s);
    default: return Q3_ERR_INVALID;
  }
}

// Shared validation and workspace carving of both decode attention entry points.
int decode_attn_setup(DecAttnArgs& a, dim3& grid, int dtype, const void* q, int64_t qsb, int64_t qsh,
                      const void* cache_k, const void* cache_v, int64_t ksb, int64_t ksh, const void* out,
                      void* workspace, int64_t B, int64_t Hq, int64_t Hkv, int64_t T_len, const int64_t* len_dev,
                      int64_t capacity, int64_t D, float scale) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && q && cache_k && cache_v && out && workspace && B > 0 &&
             Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 8 && T_len > 0 && T_len <= capacity && D == 128 &&
             B * Hkv < 65536 && decode_splits(len_dev ? capacity : T_len) <= 1024);
  Q3_REQUIRE(al16(q) && al16(cache_k) && al16(cache_v) && qsh % 8 == 0 && qsb % 8 == 0 && ksb % 8 == 0 && ksh % 8 == 0);
  // A device-resident length launches the fixed split count of the whole capacity (graph replay).
  const int64_t splits = decode_splits(len_dev ? capacity : T_len);
  a.q = (const u16*)q;
  a.qsb = qsb;
  a.qsh = qsh;
  a.ck = (u16*)cache_k;
  a.cv = (u16*)cache_v;
  a.ksb = ksb;
  a.ksh = ksh;
  a.opart = (float*)workspace;
  a.mpart = a.opart + B * Hq * splits * 128;
  a.lpart = a.mpart + B * Hq * splits;
  a.Hkv = (int)Hkv;
  a.T_len = (int)T_len;
  a.capacity = (int)capacity;
  a.splits = (int)splits;
  a.len_dev = len_dev;
  a.scale2 = scale * 1.4426950408889634f;
  grid = dim3((unsigned)splits, (unsigned)(B * Hkv));
  return 0;
}

}  // namespace

extern "C" {

int q3_gemv(int dtype, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t m, int64_t n,
            int64_t k, hipStream_t stream) {
  const void* ws[1] = {w};
  void* ys[1] = {y};
  const int64_t lds[1] = {ldy}, ns[1] = {n};
  return q3_decode_linear(dtype, x, ldx, m, k, nullptr, 0.f, 0, 1, ws, ys, lds, ns, nullptr, 0, stream);
}

int q3_decode_linear(int dtype, const void* x, int64_t ldx, int64_t m, int64_t k, const void* norm_w, float eps,
                     int mode, int nseg, const void* const* w, void* const* y, const int64_t* ldy, const int64_t* n,
                     const void* res, int64_t ldres, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && x && m >= 1 && m <= 16 && k > 0 && k % 8 == 0 &&
             k < (1 << 30) && ldx % 8 == 0 && ldx >= k && al16(x) && (!norm_w || al16(norm_w)));
  Q3_REQUIRE(w && y && ldy && n && nseg >= 1 && nseg <= 3 && (mode == 0 || mode == 1 || mode == 2));
  Q3_REQUIRE(mode != 1 || (res && ldres >= 0));
  Q3_REQUIRE(mode != 2 || (nseg == 2 && n[0] == n[1]));
  DecArgs a{};
  int64_t tiles = 0;
  for (int i = 0; i < nseg; ++i) {
    Q3_REQUIRE(w[i] && y[i] && al16(w[i]) && n[i] > 0 && n[i] < (1ll << 30) && ldy[i] >= n[i]);
    const int t = (int)((n[i] + 15) / 16);
    a.seg[i] = DecSeg{(const u16*)w[i], (u16*)y[i], ldy[i], (int)n[i], t};
    if (mode != 2 || i == 0) tiles += t;
  }
  Q3_REQUIRE(tiles < (1ll << 31));
  a.nseg = nseg;
  a.x = (const u16*)x;
  a.ldx = ldx;
  a.M = (int)m;
  a.K = (int)k;
  a.nw = (const u16*)norm_w;
  a.eps = eps;
  a.res = (const u16*)res;
  a.ldres = ldres;
  if (dtype == Q3_BF16) return dlinear_t<BF16>(a, (int)tiles, mode, norm_w != nullptr, stream);
  return dlinear_t<F16>(a, (int)tiles, mode, norm_w != nullptr, stream);
}

int q3_kv_append(int dtype, const void* k, const void* v, void* cache_k, void* cache_v, int64_t B, int64_t S,
                 int64_t H, int64_t D, int64_t capacity, int64_t start, const int64_t* start_dev,
                 hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && k && v && cache_k && cache_v && B > 0 && S > 0 && H > 0 &&
             D > 0 && D % 8 == 0 && (start_dev || (start >= 0 && start + S <= capacity)) && al16(k) && al16(v) &&
             al16(cache_k) && al16(cache_v));
  const int64_t nvec = B * S * H * (D / 8);
  kv_append_kernel<<<q3_grid_for(nvec, kThreads), kThreads, 0, stream>>>(
      (const u16*)k, (const u16*)v, (u16*)cache_k, (u16*)cache_v, (int)S, (int)H, (int)D, (int)capacity, (int)start,
      start_dev, nvec);
  return (int)hipGetLastError();
}

size_t q3_decode_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t T_len) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || T_len <= 0) return 0;
  return (size_t)(B * Hq * decode_splits(T_len)) * (128 + 2) * sizeof(float);
}

int q3_decode_attention(int dtype, const void* q, int64_t qsb, int64_t qsh, const void* cache_k, const void* cache_v,
                        int64_t ksb, int64_t ksh, void* out, int64_t osb, int64_t osh, void* workspace, int64_t B,
                        int64_t Hq, int64_t Hkv, int64_t T_len, const int64_t* len_dev, int64_t capacity, int64_t D,
                        float scale, hipStream_t stream) {
  DecAttnArgs a{};
  dim3 grid;
  const int rc = decode_attn_setup(a, grid, dtype, q, qsb, qsh, cache_k, cache_v, ksb, ksh, out, workspace, B, Hq, Hkv,
                                   T_len, len_dev, capacity, D, scale);
  if (rc) return rc;
  const int G = (int)(Hq / Hkv);
  if (dtype == Q3_BF16) return decode_t<BF16, false>(G, a, grid, out, osb, osh, stream);
  return decode_t<F16, false>(G, a, grid, out, osb, osh, stream);
}

int q3_decode_step_attention(int dtype, const void* q, int64_t qsb, int64_t qsh, const void* k, const void* v,
                             int64_t kvsb, int64_t kvsh, const void* q_norm_w, const void* k_norm_w, float eps,
                             const void* cos, const void* sin, int64_t csb, void* cache_k, void* cache_v, int64_t ksb,
                             int64_t ksh, void* out, int64_t osb, int64_t osh, void* workspace, int64_t B, int64_t Hq,
                             int64_t Hkv, int64_t T_len, const int64_t* len_dev, int64_t capacity, int64_t D,
                             float scale, hipStream_t stream) {
  DecAttnArgs a{};
  dim3 grid;
  const int rc = decode_attn_setup(a, grid, dtype, q, qsb, qsh, cache_k, cache_v, ksb, ksh, out, workspace, B, Hq, Hkv,
                                   T_len, len_dev, capacity, D, scale);
  if (rc) return rc;
  Q3_REQUIRE(k && v && q_norm_w && k_norm_w && cos && sin && al16(k) && al16(v) && al16(q_norm_w) &&
             al16(k_norm_w) && al16(cos) && al16(sin) && kvsb % 8 == 0 && kvsh % 8 == 0 && csb % 8 == 0);
  a.k = (const u16*)k;
  a.v = (const u16*)v;
  a.kvsb = kvsb;
  a.kvsh = kvsh;
  a.qw = (const u16*)q_norm_w;
  a.kw = (const u16*)k_norm_w;
  a.eps = eps;
  a.cs = (const u16*)cos;
  a.sn = (const u16*)sin;
  a.csb = csb;
  const int G = (int)(Hq / Hkv);
  if (dtype == Q3_BF16) return decode_t<BF16, true>(G, a, grid, out, osb, osh, stream);
  return decode_t<F16, true>(G, a, grid, out, osb, osh, stream);
}

}  // extern "C"

namespace {

// Split partials of q3_decode_step_attention_noalloc live in this file-scope device array instead of
// a caller workspace.  Each GPU holds its own copy (for the life of the process) at its own address.
// In host code `scratch` only names the symbol: its device address, per device, comes from
// hipGetSymbolAddress and is the only handle passed to kernels.
constexpr size_t kScratchBytes = Q3_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return Q3_ERR_INVALID;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return Q3_ERR_INVALID;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" {

int q3_decode_step_attention_noalloc(int dtype, const void* q, int64_t qsb, int64_t qsh, const void* k, const void* v,
                                     int64_t kvsb, int64_t kvsh, const void* q_norm_w, const void* k_norm_w, float eps,
                                     const void* cos, const void* sin, int64_t csb, void* cache_k, void* cache_v,
                                     int64_t ksb, int64_t ksh, void* out, int64_t osb, int64_t osh, int64_t B,
                                     int64_t Hq, int64_t Hkv, int64_t T_len, const int64_t* len_dev, int64_t capacity,
                                     int64_t D, float scale, hipStream_t stream) {
  // The partials (written in full by the split kernel before the merge reads them) must fit the array.
  const int64_t span = len_dev ? capacity : T_len;
  if (q3_decode_attention_workspace_bytes(B, Hq, Hkv, span) > kScratchBytes) return Q3_ERR_SCRATCH;
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return q3_decode_step_attention(dtype, q, qsb, qsh, k, v, kvsb, kvsh, q_norm_w, k_norm_w, eps, cos, sin, csb,
                                  cache_k, cache_v, ksb, ksh, out, osb, osh, ws, B, Hq, Hkv, T_len, len_dev, capacity,
                                  D, scale, stream);
}

size_t q3_greedy_select_workspace_bytes(int64_t batch) { return (size_t)batch * 64 * (sizeof(float) + sizeof(int)); }

int q3_greedy_select(int dtype, const void* logits, int64_t ld, int64_t batch, int64_t vocab, void* workspace,
                     int64_t* ids, int64_t ld_ids, int64_t pos, const int64_t* pos_dev, int64_t* next, uint8_t* done,
                     const int64_t* eos, int n_eos, int64_t pad, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_F32 || dtype == Q3_F16 || dtype == Q3_BF16) && logits && workspace && next && done &&
             batch > 0 && batch < 65536 && vocab > 0 && vocab < (1ll << 31) && n_eos >= 0 && (n_eos == 0 || eos));
  constexpr int parts = 64;
  float* pv = (float*)workspace;
  int* pi = (int*)(pv + batch * parts);
  dim3 g((unsigned)parts, (unsigned)batch);
  if (dtype == Q3_BF16)
    argmax_parts_kernel<BF16><<<g, kThreads, 0, stream>>>((const u16*)logits, ld, vocab, pv, pi, parts);
  else if (dtype == Q3_F16)
    argmax_parts_kernel<F16><<<g, kThreads, 0, stream>>>((const u16*)logits, ld, vocab, pv, pi, parts);
  else
    argmax_parts_kernel<F32><<<g, kThreads, 0, stream>>>((const float*)logits, ld, vocab, pv, pi, parts);
  select_kernel<<<(unsigned)((batch + 63) / 64), 64, 0, stream>>>(pv, pi, parts, ids, ld_ids, pos, pos_dev, next,
                                                                   done, eos, n_eos, pad, (int)batch);
  return (int)hipGetLastError();
}

int q3_advance(int64_t* counter, int64_t by, hipStream_t stream) {
  Q3_REQUIRE(counter);
  advance_kernel<<<1, 1, 0, stream>>>(counter, by);
  return (int)hipGetLastError();
}

}  // extern "C"

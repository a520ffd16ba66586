// RMSNorm and fused per-head RMSNorm + split-half RoPE, forward and backward.
//
// Mapping: a "row" (one token of the hidden state, or one (token, head) of Q/K) is owned by an
// aligned group of TPR lanes; lane t of the group holds the 16-byte vectors t, t+TPR, ... of the
// row in registers, so x is read from HBM exactly once per pass and every row reduction is a
// DPP/swizzle butterfly inside the group (TPR <= 64) or wave butterflies + LDS (TPR = 256).
// Weight gradients are accumulated per lane across the rows a workgroup visits, folded across the
// workgroup in a fixed order, written as one fp32 partial row per workgroup, and summed over
// workgroups by one fixed-order column-sum launch: the result is bitwise deterministic.
#include "common.h"

namespace {

constexpr int kBlock = 256;

template <int TPR> Q3_DEV float row_sum(float x, float* red) {
  if constexpr (TPR <= 64) {
    return group_sum<TPR>(x);
  } else {
    x = group_sum<64>(x);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if (lane_id() == 0) red[w] = x;
    __syncthreads();
    // the TPR / 64 waves of this thread's row group
    const float* r = red + (threadIdx.x / TPR) * (TPR / 64);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < TPR / 64; ++i) s += r[i];
    return s;
  }
}

// Two row sums at once (one pair of barriers when the row spans several waves); red holds
// 2 * kBlock / 64 floats.
template <int TPR> Q3_DEV void row_sum2(float& a, float& b, float* red) {
  if constexpr (TPR <= 64) {
    a = group_sum<TPR>(a);
    b = group_sum<TPR>(b);
  } else {
    a = group_sum<64>(a);
    b = group_sum<64>(b);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if (lane_id() == 0) {
      red[2 * w] = a;
      red[2 * w + 1] = b;
    }
    __syncthreads();
    const float* r = red + 2 * (threadIdx.x / TPR) * (TPR / 64);
    a = b = 0.f;
#pragma unroll
    for (int i = 0; i < TPR / 64; ++i) {
      a += r[2 * i];
      b += r[2 * i + 1];
    }
  }
}

// ---------------------------------------------------------------- RMSNorm forward
template <typename T, int TPR, int MAXV>
__global__ __launch_bounds__(kBlock) void rmsnorm_fwd_kernel(const typename T::storage* __restrict__ x,
                                                             const typename T::storage* __restrict__ w,
                                                             typename T::storage* __restrict__ y, int64_t rows,
                                                             int h, float eps) {
  constexpr int V = T::vec;
  constexpr int RPB = kBlock / TPR;
  __shared__ float red[kBlock / 64];
  const int nvec = h / V;
  const int t = threadIdx.x % TPR, g = threadIdx.x / TPR;
  const float inv_h = 1.f / (float)h;
  // Every load of a row is issued before any is consumed (packed operands; rows past the end and
  // vectors past h re-read a valid vector whose terms are masked).
  for (int64_t base = (int64_t)blockIdx.x * RPB; base < rows; base += (int64_t)gridDim.x * RPB) {
    const int64_t row = base + g;
    const bool valid = row < rows;
    const int64_t rc = valid ? row : rows - 1;
    i32x4 xr[MAXV], wr[MAXV];
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int vi = j * TPR + t, vc = vi < nvec ? vi : 0;
      xr[j] = *reinterpret_cast<const i32x4*>(x + rc * h + (int64_t)vc * V);
      wr[j] = *reinterpret_cast<const i32x4*>(w + (int64_t)vc * V);
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      if (j * TPR + t < nvec) {
        const Vec<T> xv = unpack_vec<T>(xr[j]);
#pragma unroll
        for (int e = 0; e < V; ++e) ss += xv.v[e] * xv.v[e];
      }
    }
    const float inv = rsqrtf(row_sum<TPR>(ss, red) * inv_h + eps);
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int vi = j * TPR + t;
      if (valid && vi < nvec) {
        const Vec<T> xv = unpack_vec<T>(xr[j]), wv = unpack_vec<T>(wr[j]);
        Vec<T> o;
#pragma unroll
        for (int e = 0; e < V; ++e) o.v[e] = xv.v[e] * inv * wv.v[e];
        store_vec<T>(y + row * h + (int64_t)vi * V, o);
      }
    }
  }
}

// ---------------------------------------------------------------- RMSNorm backward (dx + dw partials)
// RES: dx = dres + (the norm's input gradient) -- the residual branch's gradient of the same input,
// summed here instead of in a separate add.
template <typename T, int TPR, int MAXV, bool RES>
__global__ __launch_bounds__(kBlock) void rmsnorm_bwd_kernel(const typename T::storage* __restrict__ x,
                                                             const typename T::storage* __restrict__ w,
                                                             const typename T::storage* __restrict__ dy,
                                                             const typename T::storage* __restrict__ dres,
                                                             typename T::storage* __restrict__ dx,
                                                             float* __restrict__ partial, int64_t rows, int h,
                                                             float eps) {
  constexpr int V = T::vec;
  constexpr int RPB = kBlock / TPR;
  extern __shared__ float fold[];  // h floats, then the weight row (h storage elements)
  __shared__ float red[2 * (kBlock / 64)];
  const int nvec = h / V;
  const int t = threadIdx.x % TPR, g = threadIdx.x / TPR;
  const float inv_h = 1.f / (float)h;
  // Operands stay packed (16 bytes per vector) until used, and every load of a row is issued before
  // any is consumed: rows past the end and vectors past h re-read a valid vector, and their terms
  // are masked where they are used.
  // The weight row lives in LDS (read by both passes of every row), leaving the registers to the
  // row operands in flight and the fp32 dW accumulators.
  i32x4* wsh = reinterpret_cast<i32x4*>(fold + h);
  for (int i = threadIdx.x; i < nvec; i += kBlock) wsh[i] = *reinterpret_cast<const i32x4*>(w + (int64_t)i * V);
  __syncthreads();
  float acc[MAXV][V];
#pragma unroll
  for (int j = 0; j < MAXV; ++j)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[j][e] = 0.f;
  for (int64_t base = (int64_t)blockIdx.x * RPB; base < rows; base += (int64_t)gridDim.x * RPB) {
    const int64_t row = base + g;
    const bool valid = row < rows;
    const int64_t rc = valid ? row : rows - 1;
    i32x4 xr[MAXV], gr[MAXV], rr[RES ? MAXV : 1];
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int vi = j * TPR + t;
      const int64_t off = rc * h + (int64_t)(vi < nvec ? vi : 0) * V;
      // x (the forward pass's input) and dres were written long before this launch: streamed past
      // the caches.  dy was just produced by the preceding launch and may still be cache-resident.
      // [32768, 4096] bf16 on MI355X: 161 -> 143 us (62 -> 70 % of HBM bandwidth); [8192, 4096]: level.
      xr[j] = ld_nt(x + off);
      gr[j] = *reinterpret_cast<const i32x4*>(dy + off);
      if constexpr (RES) rr[j] = ld_nt(dres + off);
    }
    float ss = 0.f, dot = 0.f;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      if (j * TPR + t < nvec) {
        const Vec<T> xv = unpack_vec<T>(xr[j]), gv = unpack_vec<T>(gr[j]), wf = unpack_vec<T>(wsh[j * TPR + t]);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          ss += xv.v[e] * xv.v[e];
          dot += gv.v[e] * wf.v[e] * xv.v[e];
        }
      }
    }
    row_sum2<TPR>(ss, dot, red);
    const float inv = rsqrtf(ss * inv_h + eps);
    const float c = inv * inv * inv * dot * inv_h;  // inv * (inv^2 * mean(g*w*x))
    // The second pass unpacks the packed operands again: keeping the unpacked fp32 copies live across
    // the reductions took the kernel to 356 VGPRs (one workgroup per CU, too few loads in flight).
#pragma unroll
    for (int j = 0; j < MAXV; ++j) asm volatile("" : "+v"(xr[j]), "+v"(gr[j]));
    if constexpr (RES) {
#pragma unroll
      for (int j = 0; j < MAXV; ++j) asm volatile("" : "+v"(rr[j]));
    }
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int vi = j * TPR + t;
      if (valid && vi < nvec) {
        const Vec<T> xv = unpack_vec<T>(xr[j]), gv = unpack_vec<T>(gr[j]), wf = unpack_vec<T>(wsh[vi]);
        Vec<T> o;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          o.v[e] = gv.v[e] * wf.v[e] * inv - xv.v[e] * c;
          acc[j][e] += gv.v[e] * xv.v[e] * inv;
        }
        if constexpr (RES) {  // the norm's gradient rounded as the standalone kernel rounds it, then added
          const Vec<T> rv = unpack_vec<T>(rr[j]);
#pragma unroll
          for (int e = 0; e < V; ++e) o.v[e] = to_f32<T>(from_f32<T>(o.v[e])) + rv.v[e];
        }
        store_vec<T>(dx + row * h + (int64_t)vi * V, o);
      }
    }
  }
  // Fold the RPB row groups of this workgroup in a fixed order, then write one partial row.
  for (int gi = 0; gi < RPB; ++gi) {
    if (g == gi) {
#pragma unroll
      for (int j = 0; j < MAXV; ++j) {
        const int vi = j * TPR + t;
        if (vi < nvec) {
#pragma unroll
          for (int e = 0; e < V; ++e) {
            const int c = vi * V + e;
            fold[c] = (gi == 0) ? acc[j][e] : fold[c] + acc[j][e];
          }
        }
      }
    }
    __syncthreads();
  }
  for (int c = threadIdx.x; c < h; c += kBlock) partial[(int64_t)blockIdx.x * h + c] = fold[c];
}

// Column sums of an fp32 [R][h] partial matrix in one launch: a workgroup owns L * V columns
// (L lanes of V consecutive columns) and 256 / L row groups; row group g sums rows g, g + 256 / L,
// ... in order, then the groups fold by a lane butterfly inside each wave and through LDS across the
// waves.  Same (R, h) -> same summation order -> bitwise reproducible results.
template <typename O, int L, int V>
__global__ __launch_bounds__(kBlock) void colsum_kernel(const float* __restrict__ in,
                                                        typename O::storage* __restrict__ out, int rows, int h) {
  constexpr int RG = kBlock / L, W = L * V;
  static_assert(L <= 64 && 64 % L == 0, "row groups of one column set spread over every wave");
  __shared__ float red[kBlock / 64][W];
  const int lc = threadIdx.x % L, g = threadIdx.x / L;
  const int c0 = (blockIdx.x * L + lc) * V;
  const int cc = c0 < h ? c0 : 0;
  float s[V];
#pragma unroll
  for (int e = 0; e < V; ++e) s[e] = 0.f;
  // 8 rows in flight per step (clamped indices, masked terms)
  for (int r0 = g; r0 < rows; r0 += 8 * RG) {
    float v[8][V];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t r = min(r0 + i * RG, rows - 1);
      if constexpr (V == 4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(in + r * h + cc);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] = x[e];
      } else {
        v[i][0] = in[r * h + cc];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (r0 + i * RG < rows) {
#pragma unroll
        for (int e = 0; e < V; ++e) s[e] += v[i][e];
      }
  }
  // the row groups of a wave (lanes L apart) by a lane butterfly, then the 4 waves in order
#pragma unroll
  for (int o = L; o < 64; o <<= 1)
#pragma unroll
    for (int e = 0; e < V; ++e) s[e] += __shfl_xor(s[e], o, 64);
  const int wi = threadIdx.x >> 6;
  if ((threadIdx.x & 63) < L) {
#pragma unroll
    for (int e = 0; e < V; ++e) red[wi][lc * V + e] = s[e];
  }
  __syncthreads();
  if (threadIdx.x < L && c0 < h) {
#pragma unroll
    for (int e = 0; e < V; ++e) {
      float sum = red[0][lc * V + e];
#pragma unroll
      for (int w = 1; w < kBlock / 64; ++w) sum += red[w][lc * V + e];
      out[c0 + e] = from_f32<O>(sum);
    }
  }
}

// dw[c] = sum over the nb partial rows in `part`.
template <typename T> void colsum(float* part, typename T::storage* dw, int nb, int h, hipStream_t s) {
  if (h % 4 == 0) {
    if (h >= 1024) {
      colsum_kernel<T, 4, 4><<<(unsigned)((h + 15) / 16), kBlock, 0, s>>>(part, dw, nb, h);
    } else {
      colsum_kernel<T, 1, 4><<<(unsigned)((h + 3) / 4), kBlock, 0, s>>>(part, dw, nb, h);
    }
  } else {
    colsum_kernel<T, 4, 1><<<(unsigned)((h + 3) / 4), kBlock, 0, s>>>(part, dw, nb, h);
  }
}

// ---------------------------------------------------------------- generic (scalar) row kernels
// One wave per row, scalar element loop: any h (rmsnorm) or any even d (norm+rope).
// `heads` > 0 enables the rotation (cos/sin indexed by row / heads).
template <typename T>
__global__ __launch_bounds__(kBlock) void rownorm_generic_fwd(const typename T::storage* __restrict__ x,
                                                              const typename T::storage* __restrict__ w,
                                                              const typename T::storage* __restrict__ cs,
                                                              const typename T::storage* __restrict__ sn,
                                                              typename T::storage* __restrict__ y, int64_t rows,
                                                              int h, int heads, float eps) {
  const int64_t row = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave exits together
  const int l = lane_id();
  const typename T::storage* xr = x + row * h;
  float ss = 0.f;
  for (int e = l; e < h; e += 64) {
    const float v = to_f32<T>(xr[e]);
    ss += v * v;
  }
  const float inv = rsqrtf(group_sum<64>(ss) / (float)h + eps);
  const int half = h / 2;
  const int64_t tok = heads > 0 ? row / heads : 0;
  for (int e = l; e < h; e += 64) {
    const float n = to_f32<T>(xr[e]) * inv * to_f32<T>(w[e]);
    float o = n;
    if (heads > 0) {
      const int p = e < half ? e + half : e - half;
      const float np = to_f32<T>(xr[p]) * inv * to_f32<T>(w[p]);
      const float s = e < half ? -1.f : 1.f;
      o = n * to_f32<T>(cs[tok * h + e]) + s * np * to_f32<T>(sn[tok * h + e]);
    }
    y[row * h + e] = from_f32<T>(o);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void rownorm_generic_bwd(const typename T::storage* __restrict__ x,
                                                              const typename T::storage* __restrict__ w,
                                                              const typename T::storage* __restrict__ cs,
                                                              const typename T::storage* __restrict__ sn,
                                                              const typename T::storage* __restrict__ dy,
                                                              typename T::storage* __restrict__ dx,
                                                              float* __restrict__ partial, int64_t rows, int h,
                                                              int heads, float eps) {
  // Each workgroup owns a contiguous slab of rows; its 4 waves take rows round-robin and each wave
  // accumulates its weight-gradient row in its own partial row of global memory (L2 resident), so
  // the fixed-order column sum over all partial rows is deterministic.
  const int wv = threadIdx.x >> 6, l = lane_id();
  const int64_t per = (rows + gridDim.x - 1) / gridDim.x;
  const int64_t r0 = (int64_t)blockIdx.x * per, r1 = r0 + per < rows ? r0 + per : rows;
  const int half = h / 2;
  float* mine = partial + ((int64_t)blockIdx.x * 4 + wv) * h;
  for (int e = l; e < h; e += 64) mine[e] = 0.f;
  for (int64_t row = r0 + wv; row < r1; row += 4) {
    const int64_t tok = heads > 0 ? row / heads : 0;
    float ss = 0.f, dot = 0.f;
    for (int e = l; e < h; e += 64) {
      const float xv = to_f32<T>(x[row * h + e]);
      float g = to_f32<T>(dy[row * h + e]);
      if (heads > 0) {
        const int p = e < half ? e + half : e - half;
        const float s = e < half ? 1.f : -1.f;
        g = g * to_f32<T>(cs[tok * h + e]) + s * to_f32<T>(dy[row * h + p]) * to_f32<T>(sn[tok * h + p]);
      }
      ss += xv * xv;
      dot += g * to_f32<T>(w[e]) * xv;
    }
    ss = group_sum<64>(ss);
    dot = group_sum<64>(dot);
    const float inv = rsqrtf(ss / (float)h + eps);
    const float c = inv * inv * inv * dot / (float)h;
    for (int e = l; e < h; e += 64) {
      const float xv = to_f32<T>(x[row * h + e]);
      float g = to_f32<T>(dy[row * h + e]);
      if (heads > 0) {
        const int p = e < half ? e + half : e - half;
        const float s = e < half ? 1.f : -1.f;
        g = g * to_f32<T>(cs[tok * h + e]) + s * to_f32<T>(dy[row * h + p]) * to_f32<T>(sn[tok * h + p]);
      }
      dx[row * h + e] = from_f32<T>(g * to_f32<T>(w[e]) * inv - xv * c);
      mine[e] += g * xv * inv;
    }
  }
}

// ---------------------------------------------------------------- fused norm + rope (vector path)
// TPR = d / VEC lanes per (token, head) row, one 16-byte vector per lane; the rotation partner of
// lane t is lane t ^ (TPR/2) (requires (d/2) % VEC == 0 and TPR a power of two <= 64).
template <int TPR> Q3_DEV float partner(float v) {
  if constexpr (TPR == 16) {
    // row_ror:8 inside a 16-lane DPP row == xor 8.
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, true));
  } else {
    return __shfl_xor(v, TPR / 2, 64);
  }
}

template <typename T, int TPR>
__global__ __launch_bounds__(kBlock) void norm_rope_fwd_kernel(const typename T::storage* __restrict__ x,
                                                               const typename T::storage* __restrict__ w,
                                                               const typename T::storage* __restrict__ cs,
                                                               const typename T::storage* __restrict__ sn,
                                                               typename T::storage* __restrict__ y, int64_t rows,
                                                               int heads, float eps) {
  constexpr int V = T::vec, D = TPR * V, RPB = kBlock / TPR;
  const int t = threadIdx.x % TPR, g = threadIdx.x / TPR;
  const float sign = (t < TPR / 2) ? -1.f : 1.f;
  const Vec<T> wv = load_vec<T>(w + t * V);
  for (int64_t base = (int64_t)blockIdx.x * RPB; base < rows; base += (int64_t)gridDim.x * RPB) {
    const int64_t row = base + g;
    const bool valid = row < rows;
    const int64_t tok = row / heads;
    Vec<T> xv, cv, sv;
    float ss = 0.f;
    if (valid) {
      xv = load_vec<T>(x + row * D + t * V);
      cv = load_vec<T>(cs + tok * D + t * V);
      sv = load_vec<T>(sn + tok * D + t * V);
#pragma unroll
      for (int e = 0; e < V; ++e) ss += xv.v[e] * xv.v[e];
    }
    const float inv = rsqrtf(group_sum<TPR>(ss) * (1.f / D) + eps);
    Vec<T> o;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float n = xv.v[e] * inv * wv.v[e];
      const float np = partner<TPR>(n);
      o.v[e] = n * cv.v[e] + sign * np * sv.v[e];
    }
    if (valid) store_vec<T>(y + row * D + t * V, o);
  }
}

template <typename T, int TPR>
__global__ __launch_bounds__(kBlock) void norm_rope_bwd_kernel(const typename T::storage* __restrict__ x,
                                                               const typename T::storage* __restrict__ w,
                                                               const typename T::storage* __restrict__ cs,
                                                               const typename T::storage* __restrict__ sn,
                                                               const typename T::storage* __restrict__ dy,
                                                               typename T::storage* __restrict__ dx,
                                                               float* __restrict__ partial, int64_t rows, int heads,
                                                               float eps) {
  constexpr int V = T::vec, D = TPR * V, RPB = kBlock / TPR;
  __shared__ float fold[kBlock / 64][D];
  const int t = threadIdx.x % TPR, g = threadIdx.x / TPR;
  const float sign = (t < TPR / 2) ? 1.f : -1.f;
  const Vec<T> wv = load_vec<T>(w + t * V);
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.f;
  // U rows per thread and iteration (RPB apart), every load issued before the first use at clamped
  // row indices (rows past the end are masked at the store and in the dw sum).
  constexpr int U = 4;
  for (int64_t base = (int64_t)blockIdx.x * RPB * U; base < rows; base += (int64_t)gridDim.x * RPB * U) {
    i32x4 xr[U], gr[U], cr[U], sr[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t rc = min(base + j * RPB + g, rows - 1), tok = rc / heads;
      xr[j] = *reinterpret_cast<const i32x4*>(x + rc * D + t * V);
      gr[j] = *reinterpret_cast<const i32x4*>(dy + rc * D + t * V);
      cr[j] = *reinterpret_cast<const i32x4*>(cs + tok * D + t * V);
      sr[j] = *reinterpret_cast<const i32x4*>(sn + tok * D + t * V);
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t row = base + j * RPB + g;
      const bool valid = row < rows;
      const Vec<T> xv = unpack_vec<T>(xr[j]), gv = unpack_vec<T>(gr[j]), cv = unpack_vec<T>(cr[j]),
                   sv = unpack_vec<T>(sr[j]);
      float ss = 0.f, dot = 0.f;
      float ng[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float gs_p = partner<TPR>(gv.v[e] * sv.v[e]);  // dy[p] * sin[p]
        ng[e] = gv.v[e] * cv.v[e] + sign * gs_p;
        ss += xv.v[e] * xv.v[e];
        dot += ng[e] * wv.v[e] * xv.v[e];
      }
      ss = group_sum<TPR>(ss);
      dot = group_sum<TPR>(dot);
      const float inv = rsqrtf(ss * (1.f / D) + eps);
      const float c = inv * inv * inv * dot * (1.f / D);
      Vec<T> o;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        o.v[e] = ng[e] * wv.v[e] * inv - xv.v[e] * c;
        if (valid) acc[e] += ng[e] * xv.v[e] * inv;
      }
      if (valid) store_vec<T>(dx + row * D + t * V, o);
    }
  }
  // Fold the RPB row groups: the 64 / TPR groups of a wave by a lane butterfly, then the waves through
  // LDS in wave order (one barrier; fixed order, so the partial rows are reproducible).
#pragma unroll
  for (int o = TPR; o < 64; o <<= 1)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
  const int wi = threadIdx.x >> 6;
  if ((threadIdx.x & 63) < TPR) {
#pragma unroll
    for (int e = 0; e < V; ++e) fold[wi][t * V + e] = acc[e];
  }
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += kBlock) {
    float sum = fold[0][c];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w) sum += fold[w][c];
    partial[(int64_t)blockIdx.x * D + c] = sum;
  }
}

// ---------------------------------------------------------------- Q and K heads in one launch
// The query- and key-head halves of a layer's QK-norm + RoPE share the rotary tables and the row
// shape, so one launch covers both: workgroups [0, blocks[0]) take the query-head rows, the others
// the key-head rows (the split proportional to the row counts), each segment with its own input,
// weight, gradient and output.  Per row the arithmetic is that of norm_rope_fwd_kernel /
// norm_rope_bwd_kernel (bit-identical y and dx); each backward workgroup writes one partial row of
// 2 D floats ([dW_q | dW_k], zeros in the other segment's half), reduced by one column sum.
template <typename S> struct NrPair {
  const S* x[3];
  const S* w[2];
  const S* dy[2];
  S* y[3];  // forward output or input gradient
  int64_t rows[3];
  int heads[3];
  int blocks[3];  // workgroups per segment
  // Prefill form of the forward (CACHE): segment 1's normed + rotated keys and segment 2's values
  // (copied unchanged) go straight into the [B, heads, cap, D] caches at positions start + s of
  // [B, seq] token rows, instead of a [tokens, heads, D] output.
  int64_t cap, start, seq;
};

template <typename T, int TPR, bool CACHE>
__global__ __launch_bounds__(kBlock) void norm_rope_qk_fwd_kernel(NrPair<typename T::storage> p,
                                                                  const typename T::storage* __restrict__ cs,
                                                                  const typename T::storage* __restrict__ sn,
                                                                  float eps) {
  constexpr int V = T::vec, D = TPR * V, RPB = kBlock / TPR;
  int seg = (int)blockIdx.x >= p.blocks[0] ? 1 : 0;
  if (CACHE && (int)blockIdx.x >= p.blocks[0] + p.blocks[1]) seg = 2;
  const int blk = (int)blockIdx.x - (seg == 0 ? 0 : seg == 1 ? p.blocks[0] : p.blocks[0] + p.blocks[1]);
  const int nblk = p.blocks[seg];
  const typename T::storage* __restrict__ x = p.x[seg];
  typename T::storage* __restrict__ y = p.y[seg];
  const int64_t rows = p.rows[seg];
  const int heads = p.heads[seg];
  const int t = threadIdx.x % TPR, g = threadIdx.x / TPR;
  // output offset of a [tokens, heads] row: row-major, or its cache slot (b, head, start + s)
  auto out_off = [&](int64_t row) -> int64_t {
    if (!CACHE || seg == 0) return row * D;
    const int64_t tok = row / heads, h = row % heads, b = tok / p.seq, s = tok % p.seq;
    return ((b * heads + h) * p.cap + p.start + s) * D;
  };
  if constexpr (CACHE) {
    if (seg == 2) {  // values: copied into the cache unchanged
      for (int64_t base = (int64_t)blk * RPB; base < rows; base += (int64_t)nblk * RPB) {
        const int64_t row = base + g;
        if (row < rows)
          *reinterpret_cast<i32x4*>(y + out_off(row) + t * V) = *reinterpret_cast<const i32x4*>(x + row * D + t * V);
      }
      return;
    }
  }
  const float sign = (t < TPR / 2) ? -1.f : 1.f;
  const Vec<T> wv = load_vec<T>(p.w[seg] + t * V);
  for (int64_t base = (int64_t)blk * RPB; base < rows; base += (int64_t)nblk * RPB) {
    const int64_t row = base + g;
    const bool valid = row < rows;
    const int64_t tok = row / heads;
    Vec<T> xv, cv, sv;
    float ss = 0.f;
    if (valid) {
      xv = load_vec<T>(x + row * D + t * V);
      cv = load_vec<T>(cs + tok * D + t * V);
      sv = load_vec<T>(sn + tok * D + t * V);
#pragma unroll
      for (int e = 0; e < V; ++e) ss += xv.v[e] * xv.v[e];
    }
    const float inv = rsqrtf(group_sum<TPR>(ss) * (1.f / D) + eps);
    Vec<T> o;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float n = xv.v[e] * inv * wv.v[e];
      const float np = partner<TPR>(n);
      o.v[e] = n * cv.v[e] + sign * np * sv.v[e];
    }
    if (valid) store_vec<T>(y + out_off(row) + t * V, o);
  }
}

template <typename T, int TPR>
__global__ __launch_bounds__(kBlock) void norm_rope_qk_bwd_kernel(NrPair<typename T::storage> p,
                                                                  const typename T::storage* __restrict__ cs,
                                                                  const typename T::storage* __restrict__ sn,
                                                                  float* __restrict__ partial, float eps) {
  constexpr int V = T::vec, D = TPR * V, RPB = kBlock / TPR;
  __shared__ float fold[kBlock / 64][D];
  const int seg = (int)blockIdx.x >= p.blocks[0] ? 1 : 0;
  const int blk = (int)blockIdx.x - (seg ? p.blocks[0] : 0), nblk = p.blocks[seg];
  const typename T::storage* __restrict__ x = p.x[seg];
  const typename T::storage* __restrict__ dy = p.dy[seg];
  typename T::storage* __restrict__ dx = p.y[seg];
  const int64_t rows = p.rows[seg];
  const int heads = p.heads[seg];
  const int t = threadIdx.x % TPR, g = threadIdx.x / TPR;
  const float sign = (t < TPR / 2) ? 1.f : -1.f;
  const Vec<T> wv = load_vec<T>(p.w[seg] + t * V);
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.f;
  // U rows per thread and iteration (RPB apart), every load issued before the first use at clamped
  // row indices (rows past the end are masked at the store and in the dw sum).
  constexpr int U = 4;
  for (int64_t base = (int64_t)blk * RPB * U; base < rows; base += (int64_t)nblk * RPB * U) {
    i32x4 xr[U], gr[U], cr[U], sr[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t rc = min(base + j * RPB + g, rows - 1), tok = rc / heads;
      xr[j] = *reinterpret_cast<const i32x4*>(x + rc * D + t * V);
      gr[j] = *reinterpret_cast<const i32x4*>(dy + rc * D + t * V);
      cr[j] = *reinterpret_cast<const i32x4*>(cs + tok * D + t * V);
      sr[j] = *reinterpret_cast<const i32x4*>(sn + tok * D + t * V);
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t row = base + j * RPB + g;
      const bool valid = row < rows;
      const Vec<T> xv = unpack_vec<T>(xr[j]), gv = unpack_vec<T>(gr[j]), cv = unpack_vec<T>(cr[j]),
                   sv = unpack_vec<T>(sr[j]);
      float ss = 0.f, dot = 0.f;
      float ng[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float gs_p = partner<TPR>(gv.v[e] * sv.v[e]);  // dy[p] * sin[p]
        ng[e] = gv.v[e] * cv.v[e] + sign * gs_p;
        ss += xv.v[e] * xv.v[e];
        dot += ng[e] * wv.v[e] * xv.v[e];
      }
      ss = group_sum<TPR>(ss);
      dot = group_sum<TPR>(dot);
      const float inv = rsqrtf(ss * (1.f / D) + eps);
      const float c = inv * inv * inv * dot * (1.f / D);
      Vec<T> o;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        o.v[e] = ng[e] * wv.v[e] * inv - xv.v[e] * c;
        if (valid) acc[e] += ng[e] * xv.v[e] * inv;
      }
      if (valid) store_vec<T>(dx + row * D + t * V, o);
    }
  }
  // Fold the RPB row groups (lane butterfly inside a wave, then the waves through LDS in wave order).
#pragma unroll
  for (int o = TPR; o < 64; o <<= 1)
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
  const int wi = threadIdx.x >> 6;
  if ((threadIdx.x & 63) < TPR) {
#pragma unroll
    for (int e = 0; e < V; ++e) fold[wi][t * V + e] = acc[e];
  }
  __syncthreads();
  float* prow = partial + (int64_t)blockIdx.x * 2 * D;
  for (int c = threadIdx.x; c < D; c += kBlock) {
    float sum = fold[0][c];
#pragma unroll
    for (int w = 1; w < kBlock / 64; ++w) sum += fold[w][c];
    prow[seg * D + c] = sum;
    prow[(1 - seg) * D + c] = 0.f;
  }
}

// ---------------------------------------------------------------- host-side planning
int64_t bwd_blocks(int64_t rows, int64_t h) {
  const int64_t cap = h <= 256 ? 1024 : 512;
  return rows < cap ? (rows < 4 ? 4 : rows) : cap;  // >= 4: the scalar path writes 4 rows per workgroup
}

// Q/K pair backward: the workgroups of both segments together, split in proportion to the rows (at
// least one per segment).
int64_t qk_bwd_blocks(int64_t rq, int64_t rk, int64_t d) {
  const int64_t nb = bwd_blocks(rq + rk, d);
  return nb < 2 ? 2 : nb;
}
int64_t qk_bwd_blocks_q(int64_t rq, int64_t rk, int64_t d) {
  const int64_t nb = qk_bwd_blocks(rq, rk, d), bq = (nb * rq + (rq + rk) / 2) / (rq + rk);
  return bq < 1 ? 1 : bq > nb - 1 ? nb - 1 : bq;
}

// The scalar backward writes 4 partial rows per workgroup: a quarter of the workgroups keeps the
// workspace (bwd_blocks rows) the same for both paths.
int64_t generic_blocks(int64_t rows, int64_t h) {
  const int64_t nb = bwd_blocks(rows, h) / 4;
  return nb < 1 ? 1 : nb;
}

template <typename T, int TPR, int MAXV>
int launch_fwd(const void* x, const void* w, void* y, int64_t rows, int64_t h, float eps, hipStream_t s) {
  constexpr int RPB = kBlock / TPR;
  int64_t g = (rows + RPB - 1) / RPB;
  if (g > 256 * 16) g = 256 * 16;
  typedef typename T::storage S;
  rmsnorm_fwd_kernel<T, TPR, MAXV><<<(unsigned)g, kBlock, 0, s>>>((const S*)x, (const S*)w, (S*)y, rows, (int)h, eps);
  return (int)hipGetLastError();
}

template <typename T, int TPR, int MAXV>
int launch_bwd(const void* x, const void* w, const void* dy, const void* dres, void* dx, void* dw, float* part,
               int64_t rows, int64_t h, float eps, hipStream_t s) {
  typedef typename T::storage S;
  const int64_t nb = bwd_blocks(rows, h);
  if (dres)
    rmsnorm_bwd_kernel<T, TPR, MAXV, true><<<(unsigned)nb, kBlock, h * (sizeof(float) + sizeof(S)), s>>>(
        (const S*)x, (const S*)w, (const S*)dy, (const S*)dres, (S*)dx, part, rows, (int)h, eps);
  else
    rmsnorm_bwd_kernel<T, TPR, MAXV, false><<<(unsigned)nb, kBlock, h * (sizeof(float) + sizeof(S)), s>>>(
        (const S*)x, (const S*)w, (const S*)dy, nullptr, (S*)dx, part, rows, (int)h, eps);
  colsum<T>(part, (S*)dw, (int)nb, (int)h, s);
  return (int)hipGetLastError();
}

template <typename T>
int rms_fwd_dispatch(const void* x, const void* w, void* y, int64_t rows, int64_t h, float eps, hipStream_t s) {
  constexpr int V = T::vec;
  typedef typename T::storage S;
  const int64_t nvec = h / V;
  if (h % V == 0) {
    if (nvec <= 8) return launch_fwd<T, 8, 1>(x, w, y, rows, h, eps, s);
    if (nvec <= 16) return launch_fwd<T, 16, 1>(x, w, y, rows, h, eps, s);
    if (nvec <= 32) return launch_fwd<T, 32, 1>(x, w, y, rows, h, eps, s);
    if (nvec <= 64) return launch_fwd<T, 64, 1>(x, w, y, rows, h, eps, s);
    if (nvec <= 64 * 4) return launch_fwd<T, 64, 4>(x, w, y, rows, h, eps, s);
    if (nvec <= 64 * 8) return launch_fwd<T, 64, 8>(x, w, y, rows, h, eps, s);
    if (nvec <= 256 * 8) return launch_fwd<T, 256, 8>(x, w, y, rows, h, eps, s);
  }
  const int64_t g = (rows + 3) / 4;
  rownorm_generic_fwd<T><<<(unsigned)g, kBlock, 0, s>>>((const S*)x, (const S*)w, nullptr, nullptr, (S*)y, rows,
                                                        (int)h, 0, eps);
  return (int)hipGetLastError();
}

template <typename T>
int rms_bwd_dispatch(const void* x, const void* w, const void* dy, const void* dres, void* dx, void* dw, float* part,
                     int64_t rows, int64_t h, float eps, hipStream_t s) {
  constexpr int V = T::vec;
  typedef typename T::storage S;
  const int64_t nvec = h / V;
  if (h % V == 0) {
    if (nvec <= 8) return launch_bwd<T, 8, 1>(x, w, dy, dres, dx, dw, part, rows, h, eps, s);
    if (nvec <= 16) return launch_bwd<T, 16, 1>(x, w, dy, dres, dx, dw, part, rows, h, eps, s);
    if (nvec <= 32) return launch_bwd<T, 32, 1>(x, w, dy, dres, dx, dw, part, rows, h, eps, s);
    if (nvec <= 64) return launch_bwd<T, 64, 1>(x, w, dy, dres, dx, dw, part, rows, h, eps, s);
    if (nvec <= 64 * 4) return launch_bwd<T, 64, 4>(x, w, dy, dres, dx, dw, part, rows, h, eps, s);
    // 2 waves per row up to 512 vectors (h = 4096 in 16-bit types): half the registers of one wave per
    // row, measured 42.2 -> 39.8 us on [8192, 4096] (MI355X)
    if (nvec <= 128 * 4) return launch_bwd<T, 128, 4>(x, w, dy, dres, dx, dw, part, rows, h, eps, s);
    if (nvec <= 256 * 4) return launch_bwd<T, 256, 4>(x, w, dy, dres, dx, dw, part, rows, h, eps, s);
  }
  const int64_t gb = generic_blocks(rows, h);
  rownorm_generic_bwd<T><<<(unsigned)gb, kBlock, 0, s>>>((const S*)x, (const S*)w, nullptr, nullptr, (const S*)dy,
                                                         (S*)dx, part, rows, (int)h, 0, eps);
  colsum<T>(part, (S*)dw, (int)(4 * gb), (int)h, s);
  if (dres) {  // the scalar path adds the residual gradient with the streaming add kernel
    const int rc = (int)hipGetLastError();
    if (rc) return rc;
    return q3_add(T::code, dx, dres, dx, rows * h, s);
  }
  return (int)hipGetLastError();
}

template <typename T>
int nr_fwd_dispatch(const void* x, const void* w, const void* cs, const void* sn, void* y, int64_t rows,
                    int64_t heads, int64_t d, float eps, hipStream_t s) {
  constexpr int V = T::vec;
  typedef typename T::storage S;
  const int64_t tpr = d / V;
  auto grid = [&](int t) {
    int64_t g = (rows + kBlock / t - 1) / (kBlock / t);
    return (unsigned)(g > 256 * 16 ? 256 * 16 : g);
  };
  if (d % V == 0 && (d / 2) % V == 0) {
    if (tpr == 8) {
      norm_rope_fwd_kernel<T, 8><<<grid(8), kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs, (const S*)sn,
                                                             (S*)y, rows, (int)heads, eps);
      return (int)hipGetLastError();
    }
    if (tpr == 16) {
      norm_rope_fwd_kernel<T, 16><<<grid(16), kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs,
                                                               (const S*)sn, (S*)y, rows, (int)heads, eps);
      return (int)hipGetLastError();
    }
    if (tpr == 32) {
      norm_rope_fwd_kernel<T, 32><<<grid(32), kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs,
                                                               (const S*)sn, (S*)y, rows, (int)heads, eps);
      return (int)hipGetLastError();
    }
  }
  rownorm_generic_fwd<T><<<(unsigned)((rows + 3) / 4), kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs,
                                                                       (const S*)sn, (S*)y, rows, (int)d,
                                                                       (int)heads, eps);
  return (int)hipGetLastError();
}

template <typename T>
int nr_bwd_dispatch(const void* x, const void* w, const void* cs, const void* sn, const void* dy, void* dx, void* dw,
                    float* part, int64_t rows, int64_t heads, int64_t d, float eps, hipStream_t s) {
  constexpr int V = T::vec;
  typedef typename T::storage S;
  const int64_t tpr = d / V;
  int64_t nb = bwd_blocks(rows, d);
  bool done = false;
  if (d % V == 0 && (d / 2) % V == 0) {
    if (tpr == 8) {
      norm_rope_bwd_kernel<T, 8><<<(unsigned)nb, kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs,
                                                                  (const S*)sn, (const S*)dy, (S*)dx, part, rows,
                                                                  (int)heads, eps);
      done = true;
    } else if (tpr == 16) {
      norm_rope_bwd_kernel<T, 16><<<(unsigned)nb, kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs,
                                                                   (const S*)sn, (const S*)dy, (S*)dx, part, rows,
                                                                   (int)heads, eps);
      done = true;
    } else if (tpr == 32) {
      norm_rope_bwd_kernel<T, 32><<<(unsigned)nb, kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs,
                                                                   (const S*)sn, (const S*)dy, (S*)dx, part, rows,
                                                                   (int)heads, eps);
      done = true;
    }
  }
  if (!done) {
    const int64_t gb = generic_blocks(rows, d);
    rownorm_generic_bwd<T><<<(unsigned)gb, kBlock, 0, s>>>((const S*)x, (const S*)w, (const S*)cs, (const S*)sn,
                                                           (const S*)dy, (S*)dx, part, rows, (int)d, (int)heads, eps);
    nb = 4 * gb;
  }
  colsum<T>(part, (S*)dw, (int)nb, (int)d, s);
  return (int)hipGetLastError();
}

// Both Q/K launches need the vector path (d / 2 a multiple of the vector width, 8 / 16 / 32 lanes
// per row); other shapes return Q3_ERR_INVALID and the caller runs the two single-tensor launches.
template <typename T>
int nr_qk_fwd_dispatch(const NrPair<typename T::storage>& p, const void* cs, const void* sn, int64_t d, float eps,
                       hipStream_t s) {
  constexpr int V = T::vec;
  typedef typename T::storage S;
  const int64_t tpr = d / V;
  if (d % V != 0 || (d / 2) % V != 0 || (tpr != 8 && tpr != 16 && tpr != 32)) return Q3_ERR_INVALID;
  // each segment's grid as its single-tensor launch sizes it
  NrPair<S> q = p;
  const int nseg = p.cap > 0 ? 3 : 2;
  for (int i = 0; i < nseg; ++i) {
    const int64_t g = (p.rows[i] + kBlock / tpr - 1) / (kBlock / tpr);
    q.blocks[i] = (int)(g > 256 * 16 ? 256 * 16 : g);
  }
  const unsigned grid = (unsigned)(q.blocks[0] + q.blocks[1] + (nseg == 3 ? q.blocks[2] : 0));
  const S* c = (const S*)cs;
  const S* n = (const S*)sn;
  if (nseg == 3) {
    if (tpr == 8) norm_rope_qk_fwd_kernel<T, 8, true><<<grid, kBlock, 0, s>>>(q, c, n, eps);
    else if (tpr == 16) norm_rope_qk_fwd_kernel<T, 16, true><<<grid, kBlock, 0, s>>>(q, c, n, eps);
    else norm_rope_qk_fwd_kernel<T, 32, true><<<grid, kBlock, 0, s>>>(q, c, n, eps);
  } else {
    if (tpr == 8) norm_rope_qk_fwd_kernel<T, 8, false><<<grid, kBlock, 0, s>>>(q, c, n, eps);
    else if (tpr == 16) norm_rope_qk_fwd_kernel<T, 16, false><<<grid, kBlock, 0, s>>>(q, c, n, eps);
    else norm_rope_qk_fwd_kernel<T, 32, false><<<grid, kBlock, 0, s>>>(q, c, n, eps);
  }
  return (int)hipGetLastError();
}

template <typename T>
int nr_qk_bwd_dispatch(const NrPair<typename T::storage>& p, const void* cs, const void* sn, void* dw, float* part,
                       int64_t d, float eps, hipStream_t s) {
  constexpr int V = T::vec;
  typedef typename T::storage S;
  const int64_t tpr = d / V, nb = qk_bwd_blocks(p.rows[0], p.rows[1], d);
  if (d % V != 0 || (d / 2) % V != 0 || (tpr != 8 && tpr != 16 && tpr != 32)) return Q3_ERR_INVALID;
  NrPair<S> q = p;
  q.blocks[0] = (int)qk_bwd_blocks_q(p.rows[0], p.rows[1], d);
  q.blocks[1] = (int)(nb - q.blocks[0]);
  if (tpr == 8) norm_rope_qk_bwd_kernel<T, 8><<<(unsigned)nb, kBlock, 0, s>>>(q, (const S*)cs, (const S*)sn, part, eps);
  else if (tpr == 16)
    norm_rope_qk_bwd_kernel<T, 16><<<(unsigned)nb, kBlock, 0, s>>>(q, (const S*)cs, (const S*)sn, part, eps);
  else norm_rope_qk_bwd_kernel<T, 32><<<(unsigned)nb, kBlock, 0, s>>>(q, (const S*)cs, (const S*)sn, part, eps);
  colsum<T>(part, (S*)dw, (int)nb, (int)(2 * d), s);
  return (int)hipGetLastError();
}

template <typename T>
int nr_qk_cache_fwd_t(const void* q, const void* k, const void* v, const void* wq, const void* wk, const void* cs,
                      const void* sn, void* yq, void* ck, void* cv, int64_t B, int64_t S_, int64_t hq, int64_t hk,
                      int64_t d, int64_t cap, int64_t start, float eps, hipStream_t s) {
  typedef typename T::storage S;
  NrPair<S> p{};
  p.x[0] = (const S*)q;
  p.x[1] = (const S*)k;
  p.x[2] = (const S*)v;
  p.w[0] = (const S*)wq;
  p.w[1] = (const S*)wk;
  p.y[0] = (S*)yq;
  p.y[1] = (S*)ck;
  p.y[2] = (S*)cv;
  p.rows[0] = B * S_ * hq;
  p.rows[1] = p.rows[2] = B * S_ * hk;
  p.heads[0] = (int)hq;
  p.heads[1] = p.heads[2] = (int)hk;
  p.cap = cap;
  p.start = start;
  p.seq = S_;
  return nr_qk_fwd_dispatch<T>(p, cs, sn, d, eps, s);
}

template <typename T>
int nr_qk_fwd_t(const void* q, const void* k, const void* wq, const void* wk, const void* cs, const void* sn, void* yq,
                void* yk, int64_t tokens, int64_t hq, int64_t hk, int64_t d, float eps, hipStream_t s) {
  typedef typename T::storage S;
  NrPair<S> p{};
  p.x[0] = (const S*)q;
  p.x[1] = (const S*)k;
  p.w[0] = (const S*)wq;
  p.w[1] = (const S*)wk;
  p.y[0] = (S*)yq;
  p.y[1] = (S*)yk;
  p.rows[0] = tokens * hq;
  p.rows[1] = tokens * hk;
  p.heads[0] = (int)hq;
  p.heads[1] = (int)hk;
  return nr_qk_fwd_dispatch<T>(p, cs, sn, d, eps, s);
}

template <typename T>
int nr_qk_bwd_t(const void* q, const void* k, const void* wq, const void* wk, const void* cs, const void* sn,
                const void* dyq, const void* dyk, void* dxq, void* dxk, void* dw, float* part, int64_t tokens,
                int64_t hq, int64_t hk, int64_t d, float eps, hipStream_t s) {
  typedef typename T::storage S;
  NrPair<S> p{};
  p.x[0] = (const S*)q;
  p.x[1] = (const S*)k;
  p.w[0] = (const S*)wq;
  p.w[1] = (const S*)wk;
  p.dy[0] = (const S*)dyq;
  p.dy[1] = (const S*)dyk;
  p.y[0] = (S*)dxq;
  p.y[1] = (S*)dxk;
  p.rows[0] = tokens * hq;
  p.rows[1] = tokens * hk;
  p.heads[0] = (int)hq;
  p.heads[1] = (int)hk;
  return nr_qk_bwd_dispatch<T>(p, cs, sn, dw, part, d, eps, s);
}

bool dtype_ok(int dt) { return dt == Q3_F32 || dt == Q3_F16 || dt == Q3_BF16; }

}  // namespace

#define Q3_DISPATCH(dt, FN, ...)                                 \
  ((dt) == Q3_BF16 ? FN<BF16>(__VA_ARGS__)                       \
                   : (dt) == Q3_F16 ? FN<F16>(__VA_ARGS__) : FN<F32>(__VA_ARGS__))

extern "C" {

int q3_rmsnorm_fwd(int dtype, const void* x, const void* w, void* y, int64_t rows, int64_t h, float eps,
                   hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && w && y && rows > 0 && h > 0 && h <= (1 << 20) && eps > 0.f);
  return Q3_DISPATCH(dtype, rms_fwd_dispatch, x, w, y, rows, h, eps, stream);
}

size_t q3_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t h) {
  const int64_t nb = bwd_blocks(rows, h);
  return (size_t)nb * (size_t)h * sizeof(float);
}

int q3_rmsnorm_bwd(int dtype, const void* x, const void* w, const void* dy, void* dx, void* dw, void* workspace,
                   int64_t rows, int64_t h, float eps, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && w && dy && dx && dw && workspace && rows > 0 && h > 0 && eps > 0.f);
  // The vector path (h <= 8192 in 16-bit types, 4096 in fp32) folds dW in LDS; wider rows take the
  // scalar path, whose partials live in the workspace.
  Q3_REQUIRE(h <= (1 << 20));
  return Q3_DISPATCH(dtype, rms_bwd_dispatch, x, w, dy, nullptr, dx, dw, (float*)workspace, rows, h, eps, stream);
}

int q3_rmsnorm_bwd_add(int dtype, const void* x, const void* w, const void* dy, const void* dres, void* dx, void* dw,
                       void* workspace, int64_t rows, int64_t h, float eps, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && w && dy && dres && dx && dw && workspace && rows > 0 && h > 0 && eps > 0.f);
  Q3_REQUIRE(h <= (1 << 20));
  return Q3_DISPATCH(dtype, rms_bwd_dispatch, x, w, dy, dres, dx, dw, (float*)workspace, rows, h, eps, stream);
}

int q3_norm_rope_fwd(int dtype, const void* x, const void* w, const void* cos, const void* sin, void* y,
                     int64_t tokens, int64_t heads, int64_t d, float eps, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && w && cos && sin && y && tokens > 0 && heads > 0 && d > 0 && d % 2 == 0 &&
             d <= 4096 && eps > 0.f);
  return Q3_DISPATCH(dtype, nr_fwd_dispatch, x, w, cos, sin, y, tokens * heads, heads, d, eps, stream);
}

size_t q3_norm_rope_bwd_workspace_bytes(int64_t tokens, int64_t heads, int64_t d) {
  const int64_t nb = bwd_blocks(tokens * heads, d);
  return (size_t)nb * (size_t)d * sizeof(float);
}

int q3_norm_rope_bwd(int dtype, const void* x, const void* w, const void* cos, const void* sin, const void* dy,
                     void* dx, void* dw, void* workspace, int64_t tokens, int64_t heads, int64_t d, float eps,
                     hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && w && cos && sin && dy && dx && dw && workspace && tokens > 0 && heads > 0 &&
             d > 0 && d % 2 == 0 && d <= 4096 && eps > 0.f);
  return Q3_DISPATCH(dtype, nr_bwd_dispatch, x, w, cos, sin, dy, dx, dw, (float*)workspace, tokens * heads, heads, d,
                     eps, stream);
}

int q3_norm_rope_qk_fwd(int dtype, const void* q, const void* k, const void* wq, const void* wk, const void* cos,
                        const void* sin, void* yq, void* yk, int64_t tokens, int64_t hq, int64_t hk, int64_t d,
                        float eps, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && q && k && wq && wk && cos && sin && yq && yk && tokens > 0 && hq > 0 && hk > 0 &&
             d > 0 && d % 2 == 0 && d <= 4096 && eps > 0.f && tokens * (hq + hk) < (1ll << 40));
  return Q3_DISPATCH(dtype, nr_qk_fwd_t, q, k, wq, wk, cos, sin, yq, yk, tokens, hq, hk, d, eps, stream);
}

int q3_norm_rope_qk_cache_fwd(int dtype, const void* q, const void* k, const void* v, const void* wq, const void* wk,
                              const void* cos, const void* sin, void* yq, void* cache_k, void* cache_v, int64_t B,
                              int64_t S, int64_t hq, int64_t hk, int64_t d, int64_t capacity, int64_t start, float eps,
                              hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && q && k && v && wq && wk && cos && sin && yq && cache_k && cache_v && B > 0 && S > 0 &&
             hq > 0 && hk > 0 && d > 0 && d % 2 == 0 && d <= 4096 && eps > 0.f && start >= 0 && start + S <= capacity &&
             B * S * (hq + hk) < (1ll << 40) && B * hk * capacity * d < (1ll << 40));
  Q3_REQUIRE((((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)yq | (uintptr_t)cache_k |
               (uintptr_t)cache_v) & 15) == 0);
  return Q3_DISPATCH(dtype, nr_qk_cache_fwd_t, q, k, v, wq, wk, cos, sin, yq, cache_k, cache_v, B, S, hq, hk, d,
                     capacity, start, eps, stream);
}

size_t q3_norm_rope_qk_bwd_workspace_bytes(int64_t tokens, int64_t hq, int64_t hk, int64_t d) {
  if (tokens <= 0 || hq <= 0 || hk <= 0 || d <= 0) return 0;
  const int64_t nb = qk_bwd_blocks(tokens * hq, tokens * hk, d);
  return (size_t)nb * (size_t)(2 * d) * sizeof(float);
}

int q3_norm_rope_qk_bwd(int dtype, const void* q, const void* k, const void* wq, const void* wk, const void* cos,
                        const void* sin, const void* dyq, const void* dyk, void* dxq, void* dxk, void* dw,
                        void* workspace, int64_t tokens, int64_t hq, int64_t hk, int64_t d, float eps,
                        hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && q && k && wq && wk && cos && sin && dyq && dyk && dxq && dxk && dw && workspace &&
             tokens > 0 && hq > 0 && hk > 0 && d > 0 && d % 2 == 0 && d <= 4096 && eps > 0.f &&
             tokens * (hq + hk) < (1ll << 40));
  return Q3_DISPATCH(dtype, nr_qk_bwd_t, q, k, wq, wk, cos, sin, dyq, dyk, dxq, dxk, dw, (float*)workspace, tokens,
                     hq, hk, d, eps, stream);
}

}  // extern "C"

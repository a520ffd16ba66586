// Streaming kernels: RoPE tables/apply, SwiGLU fwd/bwd, residual add, cast, fill, positions,
// transpose, embedding gather and its deterministic scatter-sum.
//
// All are HBM-bound: each thread moves whole 16-byte vectors (8 x 16-bit / 4 x fp32) with a
// grid-stride loop sized to fill the 256 CUs, and falls back to scalar code only for tails or
// shapes that break 16-byte alignment.
#include "common.h"

namespace {

constexpr int kBlock = 256;

Q3_DEV float sigmoid(float g) { return q3_sigmoid(g); }

template <typename T> bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---------------------------------------------------------------- SwiGLU
// Each thread owns U 16-byte vectors per operand (kBlock apart) and issues every load before the
// first use: the sigmoid's transcendental latency then overlaps U vectors' worth of loads instead of
// serialising a load -> math -> store chain per vector (5.4 -> 6+ TB/s measured).
constexpr int kU = 4;
template <typename T>
__global__ __launch_bounds__(kBlock) void swiglu_fwd_kernel(const typename T::storage* __restrict__ g,
                                                            const typename T::storage* __restrict__ u,
                                                            typename T::storage* __restrict__ y, int64_t n,
                                                            int vec_ok) {
  constexpr int V = T::vec;
  const int64_t nv = vec_ok ? n / V : 0;
  const int64_t step = (int64_t)gridDim.x * kBlock * kU;
  for (int64_t i0 = (int64_t)blockIdx.x * kBlock * kU + threadIdx.x; i0 < nv; i0 += step) {
    i32x4 gr[kU], ur[kU];
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int64_t i = min(i0 + (int64_t)j * kBlock, nv - 1);  // clamped: loads never wait on a branch
      gr[j] = ld_nt(g + i * V);
      ur[j] = ld_nt(u + i * V);
    }
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int64_t i = i0 + (int64_t)j * kBlock;
      const Vec<T> gv = unpack_vec<T>(gr[j]), uv = unpack_vec<T>(ur[j]);
      Vec<T> o;
#pragma unroll
      for (int e = 0; e < V; ++e) o.v[e] = gv.v[e] * sigmoid(gv.v[e]) * uv.v[e];
      if (i < nv) st_nt<T>(y + i * V, o);
    }
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock) {
    const float gg = to_f32<T>(g[i]);
    y[i] = from_f32<T>(gg * sigmoid(gg) * to_f32<T>(u[i]));
  }
}

// Workgroups for one pass of kU vectors per thread over nvec vectors (a grid-stride remainder pass
// would run with part of the threads idle).
static inline unsigned one_pass_grid(int64_t nvec) {
  const int64_t g = (nvec + (int64_t)kBlock * kU - 1) / ((int64_t)kBlock * kU);
  return (unsigned)(g < 1 ? 1 : (g > 0x7fffffff ? 0x7fffffff : g));
}

template <typename T>
Q3_DEV void swiglu_grad8(const i32x4& g, const i32x4& u, const i32x4& d, Vec<T>& og, Vec<T>& ou) {
  const Vec<T> gv = unpack_vec<T>(g), uv = unpack_vec<T>(u), dv = unpack_vec<T>(d);
#pragma unroll
  for (int e = 0; e < T::vec; ++e) {
    const float s = sigmoid(gv.v[e]);
    og.v[e] = dv.v[e] * uv.v[e] * s * (1.f + gv.v[e] * (1.f - s));
    ou.v[e] = dv.v[e] * gv.v[e] * s;
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void swiglu_bwd_kernel(const typename T::storage* __restrict__ g,
                                                            const typename T::storage* __restrict__ u,
                                                            const typename T::storage* __restrict__ dy,
                                                            typename T::storage* __restrict__ dg,
                                                            typename T::storage* __restrict__ du, int64_t n,
                                                            int vec_ok) {
  constexpr int V = T::vec;
  const int64_t nv = vec_ok ? n / V : 0;
  const int64_t step = (int64_t)gridDim.x * kBlock * kU;
  for (int64_t i0 = (int64_t)blockIdx.x * kBlock * kU + threadIdx.x; i0 < nv; i0 += step) {
    i32x4 gr[kU], ur[kU], dr[kU];
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int64_t i = min(i0 + (int64_t)j * kBlock, nv - 1);
      gr[j] = ld_nt(g + i * V);
      ur[j] = ld_nt(u + i * V);
      dr[j] = ld_nt(dy + i * V);
    }
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int64_t i = i0 + (int64_t)j * kBlock;
      Vec<T> og, ou;
      swiglu_grad8<T>(gr[j], ur[j], dr[j], og, ou);
      if (i < nv) {
        st_nt<T>(dg + i * V, og);
        st_nt<T>(du + i * V, ou);
      }
    }
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock) {
    const float gg = to_f32<T>(g[i]), uu = to_f32<T>(u[i]), d = to_f32<T>(dy[i]);
    const float s = sigmoid(gg);
    dg[i] = from_f32<T>(d * uu * s * (1.f + gg * (1.f - s)));
    du[i] = from_f32<T>(d * gg * s);
  }
}

// ---------------------------------------------------------------- add / cast / fill
template <typename T>
__global__ __launch_bounds__(kBlock) void add_kernel(const typename T::storage* __restrict__ a,
                                                     const typename T::storage* __restrict__ b,
                                                     typename T::storage* __restrict__ c, int64_t n, int vec_ok) {
  constexpr int V = T::vec;
  const int64_t nv = vec_ok ? n / V : 0;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < nv; i += stride) {
    Vec<T> av = load_vec<T>(a + i * V), bv = load_vec<T>(b + i * V), o;
#pragma unroll
    for (int e = 0; e < V; ++e) o.v[e] = av.v[e] + bv.v[e];
    store_vec<T>(c + i * V, o);
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    c[i] = from_f32<T>(to_f32<T>(a[i]) + to_f32<T>(b[i]));
}

template <typename S, typename D>
__global__ __launch_bounds__(kBlock) void cast_kernel(const typename S::storage* __restrict__ x,
                                                      typename D::storage* __restrict__ y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    y[i] = from_f32<D>(to_f32<S>(x[i]));
}

template <typename T>
__global__ __launch_bounds__(kBlock) void fill_kernel(typename T::storage* __restrict__ x, float value, int64_t n) {
  const typename T::storage v = from_f32<T>(value);
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) x[i] = v;
}

__global__ __launch_bounds__(kBlock) void positions_kernel(int64_t* __restrict__ out, int64_t n, int64_t seq,
                                                           int64_t start, const int64_t* start_dev) {
  if (start_dev) start += *start_dev;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) out[i] = start + i % seq;
}

// ---------------------------------------------------------------- RoPE
// cos/sin tables: one thread per (position, j < d/2); writes columns j and j + d/2.
template <typename T>
__global__ __launch_bounds__(kBlock) void rope_tables_kernel(const void* __restrict__ pos, int pos64,
                                                             const float* __restrict__ inv_freq,
                                                             typename T::storage* __restrict__ cs,
                                                             typename T::storage* __restrict__ sn, int64_t npos,
                                                             int half) {
  const int64_t n = npos * half;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const int64_t t = i / half;
    const int j = (int)(i % half);
    const float p = pos64 ? (float)((const int64_t*)pos)[t] : (float)((const int*)pos)[t];
    const float ang = p * inv_freq[j];
    float s, c;
    sincosf(ang, &s, &c);
    const int64_t o = t * 2 * half + j;
    cs[o] = from_f32<T>(c);
    cs[o + half] = from_f32<T>(c);
    sn[o] = from_f32<T>(s);
    sn[o + half] = from_f32<T>(s);
  }
}

// Token index of a row for the two layouts: 0 = [B,S,H,D] (row = (b*S+s)*H+h),
// 1 = [B,H,S,D] (row = (b*H+h)*S+s).  cos/sin are [B*S, D].
Q3_DEV int64_t rope_token(int64_t row, int64_t seq, int64_t heads, int layout) {
  if (layout == 0) return row / heads;
  return (row / (heads * seq)) * seq + row % seq;
}

// One thread per (row, vector j of the first half): handles the element pairs (d, d + D/2).
template <typename T>
__global__ __launch_bounds__(kBlock) void rope_apply_vec_kernel(const typename T::storage* __restrict__ x,
                                                                const typename T::storage* __restrict__ cs,
                                                                const typename T::storage* __restrict__ sn,
                                                                typename T::storage* __restrict__ y, int64_t rows,
                                                                int64_t seq, int64_t heads, int d, int layout,
                                                                int backward) {
  constexpr int V = T::vec;
  const int half = d / 2, hv = half / V;
  const int64_t n = rows * hv;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const int64_t row = i / hv;
    const int j = (int)(i % hv) * V;
    const int64_t tok = rope_token(row, seq, heads, layout);
    const typename T::storage* xr = x + row * d;
    const Vec<T> a = load_vec<T>(xr + j), b = load_vec<T>(xr + half + j);
    const Vec<T> ca = load_vec<T>(cs + tok * d + j), cb = load_vec<T>(cs + tok * d + half + j);
    const Vec<T> sa = load_vec<T>(sn + tok * d + j), sb = load_vec<T>(sn + tok * d + half + j);
    Vec<T> oa, ob;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      if (!backward) {
        oa.v[e] = a.v[e] * ca.v[e] - b.v[e] * sa.v[e];
        ob.v[e] = b.v[e] * cb.v[e] + a.v[e] * sb.v[e];
      } else {
        oa.v[e] = a.v[e] * ca.v[e] + b.v[e] * sb.v[e];
        ob.v[e] = b.v[e] * cb.v[e] - a.v[e] * sa.v[e];
      }
    }
    store_vec<T>(y + row * d + j, oa);
    store_vec<T>(y + row * d + half + j, ob);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void rope_apply_scalar_kernel(const typename T::storage* __restrict__ x,
                                                                   const typename T::storage* __restrict__ cs,
                                                                   const typename T::storage* __restrict__ sn,
                                                                   typename T::storage* __restrict__ y, int64_t rows,
                                                                   int64_t seq, int64_t heads, int d, int layout,
                                                                   int backward) {
  const int half = d / 2;
  const int64_t n = rows * half;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const int64_t row = i / half;
    const int j = (int)(i % half);
    const int64_t tok = rope_token(row, seq, heads, layout);
    const float a = to_f32<T>(x[row * d + j]), b = to_f32<T>(x[row * d + half + j]);
    const float ca = to_f32<T>(cs[tok * d + j]), cb = to_f32<T>(cs[tok * d + half + j]);
    const float sa = to_f32<T>(sn[tok * d + j]), sb = to_f32<T>(sn[tok * d + half + j]);
    float oa, ob;
    if (!backward) {
      oa = a * ca - b * sa;
      ob = b * cb + a * sb;
    } else {
      oa = a * ca + b * sb;
      ob = b * cb - a * sa;
    }
    y[row * d + j] = from_f32<T>(oa);
    y[row * d + half + j] = from_f32<T>(ob);
  }
}

// ---------------------------------------------------------------- transpose
// y[b][c][r] = x[b][r][c] through a 64x64 LDS tile (row padded to 66 elements: the column reads
// of the store phase hit distinct banks).  Elements are moved as raw 16- or 32-bit words.  Output
// rows have stride ldy >= rows; the pad columns [rows, ldy) are written with zeros.
template <typename W>
__global__ __launch_bounds__(kBlock) void transpose_kernel(const W* __restrict__ x, W* __restrict__ y, int64_t rows,
                                                           int64_t cols, int64_t ldy) {
  __shared__ W tile[64][66];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const W* xb = x + b * rows * cols;
  W* yb = y + b * cols * ldy;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = xb[gr * cols + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int64_t gc = c0 + c, gr = r0 + tx;
    if (gc < cols && gr < ldy) yb[gc * ldy + gr] = gr < rows ? tile[tx][c] : (W)0;
  }
}

// 16-bit transpose without LDS: each lane loads an 8x8 block as eight 16-byte row vectors,
// transposes it in registers and stores eight 16-byte vectors.  Within a wave, lane = 8 * g + c
// covers input rows r0 + 8g..+7 and columns c0 + 8c..+7, so both the loads (8 lanes per input row)
// and the stores (8 lanes per output row) move 128 contiguous bytes.  A workgroup (4 waves) covers
// 64 rows x 256 columns.  Needs cols % 8 == 0, ldy % 8 == 0 and 16-byte aligned pointers; rows past
// `rows` (up to ldy) are written as zeros.
__global__ __launch_bounds__(kBlock) void transpose16_kernel(const u16* __restrict__ x, u16* __restrict__ y,
                                                             int64_t rows, int64_t cols, int64_t ldy) {
  const int64_t b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.y * 64 + 8 * (lane >> 3);
  const int64_t c = (int64_t)blockIdx.x * 256 + wave * 64 + 8 * (lane & 7);
  if (c >= cols || r >= ldy) return;
  const u16* xb = x + b * rows * cols + c;
  uint32_t in[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    i32x4 v = {0, 0, 0, 0};
    if (r + i < rows) v = *reinterpret_cast<const i32x4*>(xb + (r + i) * cols);
#pragma unroll
    for (int w = 0; w < 4; ++w) in[i][w] = (uint32_t)v[w];
  }
  u16* yb = y + b * cols * ldy + c * ldy + r;
#pragma unroll
  for (int j = 0; j < 8; ++j) {  // output row c + j holds element j of every input row
    const int w = j >> 1, sh = (j & 1) * 16;
    i32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = (int)(((in[2 * k][w] >> sh) & 0xffffu) | (((in[2 * k + 1][w] >> sh) & 0xffffu) << 16));
    *reinterpret_cast<i32x4*>(yb + (int64_t)j * ldy) = o;
  }
}

// ---------------------------------------------------------------- row-strided variants
// The same element maps on [rows, cols] blocks whose rows sit at their own strides, so gate/up (or
// q/k/v) results can live side by side in one [rows, 2 cols] buffer.  16-byte vectors when cols and
// every stride are multiples of 8 elements and the pointers 16-byte aligned, else scalar.
template <typename T>
__global__ __launch_bounds__(kBlock) void swiglu_bwd2d_kernel(const typename T::storage* __restrict__ g, int64_t ldg,
                                                              const typename T::storage* __restrict__ u, int64_t ldu,
                                                              const typename T::storage* __restrict__ dy,
                                                              int64_t lddy, typename T::storage* __restrict__ dg,
                                                              int64_t lddg, typename T::storage* __restrict__ du,
                                                              int64_t lddu, int64_t rows, int64_t cols, int vec) {
  if (vec) {  // U vectors per thread, every load issued first (index math in 32 bits: n < 2^31)
    const int per = (int)(cols / T::vec), n = (int)(rows * per);
    const int step = gridDim.x * kBlock * kU;
    for (int i0 = blockIdx.x * kBlock * kU + threadIdx.x; i0 < n; i0 += step) {
      i32x4 gr[kU], ur[kU], dr[kU];
      int64_t rr[kU];
      int cc[kU];
#pragma unroll
      for (int j = 0; j < kU; ++j) {
        const int i = min(i0 + j * kBlock, n - 1);
        rr[j] = i / per;
        cc[j] = (i % per) * T::vec;
        gr[j] = ld_nt(g + rr[j] * ldg + cc[j]);
        ur[j] = ld_nt(u + rr[j] * ldu + cc[j]);
        dr[j] = ld_nt(dy + rr[j] * lddy + cc[j]);
      }
#pragma unroll
      for (int j = 0; j < kU; ++j) {
        Vec<T> og, ou;
        swiglu_grad8<T>(gr[j], ur[j], dr[j], og, ou);
        if (i0 + j * kBlock < n) {
          st_nt<T>(dg + rr[j] * lddg + cc[j], og);
          st_nt<T>(du + rr[j] * lddu + cc[j], ou);
        }
      }
    }
    return;
  }
  const int64_t n = rows * cols;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / cols, c = i % cols;
    const float gg = to_f32<T>(g[r * ldg + c]), uu = to_f32<T>(u[r * ldu + c]), d = to_f32<T>(dy[r * lddy + c]);
    const float sg = sigmoid(gg);
    dg[r * lddg + c] = from_f32<T>(d * uu * sg * (1.f + gg * (1.f - sg)));
    du[r * lddu + c] = from_f32<T>(d * gg * sg);
  }
}

template <typename S>
__global__ __launch_bounds__(kBlock) void copy2d_kernel(const S* __restrict__ x, int64_t ldx, S* __restrict__ y,
                                                        int64_t ldy, int64_t rows, int64_t cols, int vec) {
  constexpr int V = 16 / sizeof(S);
  const int64_t per = vec ? cols / V : cols, n = rows * per;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / per, c = i % per;
    if (vec)
      *reinterpret_cast<i32x4*>(y + r * ldy + c * V) = *reinterpret_cast<const i32x4*>(x + r * ldx + c * V);
    else
      y[r * ldy + c] = x[r * ldx + c];
  }
}

// y[c * ldy + r] = x[r * ldx + c] for r < rows, c < cols; nothing else is written.  16-bit vector
// path: the 8x8 register-block kernel above with an input row stride (rows % 8 == 0 so no block
// reaches past the last row).
__global__ __launch_bounds__(kBlock) void transpose2d16_kernel(const u16* __restrict__ x, int64_t ldx,
                                                               u16* __restrict__ y, int64_t ldy, int64_t rows,
                                                               int64_t cols) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.y * 64 + 8 * (lane >> 3);
  const int64_t c = (int64_t)blockIdx.x * 256 + wave * 64 + 8 * (lane & 7);
  if (c >= cols || r >= rows) return;
  uint32_t in[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const i32x4 v = *reinterpret_cast<const i32x4*>(x + (r + i) * ldx + c);
#pragma unroll
    for (int w = 0; w < 4; ++w) in[i][w] = (uint32_t)v[w];
  }
  u16* yb = y + c * ldy + r;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int w = j >> 1, sh = (j & 1) * 16;
    i32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = (int)(((in[2 * k][w] >> sh) & 0xffffu) | (((in[2 * k + 1][w] >> sh) & 0xffffu) << 16));
    *reinterpret_cast<i32x4*>(yb + (int64_t)j * ldy) = o;
  }
}

// 16-bit transpose of full 128 x 128 tiles through LDS: rows go in as 256-byte row segments and come
// out as 256-byte row segments of y (the register-block kernel above moves 128-byte segments).  LDS
// row r keeps its 16-byte chunk c at physical chunk c ^ ((r >> 3) & 15): the row writes and the
// column gathers (16 lanes on rows 8 apart) both hit 16 different chunks.
__global__ __launch_bounds__(kBlock) void transpose2d16_lds_kernel(const u16* __restrict__ x, int64_t ldx,
                                                                   u16* __restrict__ y, int64_t ldy, int64_t bsx,
                                                                   int64_t bsy) {
  __shared__ __attribute__((aligned(16))) u16 tile[128 * 128];
  const int t = threadIdx.x, ch = t & 15, rr = t >> 4;
  const int64_t r0 = (int64_t)blockIdx.y * 128, c0 = (int64_t)blockIdx.x * 128;
  x += (int64_t)blockIdx.z * bsx;  // batch z: x [rows, cols] at z bsx, y [cols, ldy] at z bsy
  y += (int64_t)blockIdx.z * bsy;
  i32x4 v[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) v[p] = *reinterpret_cast<const i32x4*>(x + (r0 + 16 * p + rr) * ldx + c0 + 8 * ch);
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int r = 16 * p + rr;
    *reinterpret_cast<i32x4*>(tile + r * 128 + 8 * (ch ^ ((r >> 3) & 15))) = v[p];
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 8; ++p) {  // output row oc (a tile column), rows 8 ch .. 8 ch + 7 of the tile
    const int oc = 16 * p + rr, pc = (oc >> 3), off = oc & 7;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ra = 8 * ch + 2 * e, rb = ra + 1;  // (ra >> 3) & 15 == ch for both rows
      const uint32_t a = tile[ra * 128 + 8 * (pc ^ ch) + off], b = tile[rb * 128 + 8 * (pc ^ ch) + off];
      w[e] = a | (b << 16);
    }
    *reinterpret_cast<i32x4*>(y + (c0 + oc) * ldy + r0 + 8 * ch) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

template <typename S>
__global__ __launch_bounds__(kBlock) void transpose2d_scalar_kernel(const S* __restrict__ x, int64_t ldx,
                                                                    S* __restrict__ y, int64_t ldy, int64_t rows,
                                                                    int64_t cols) {
  __shared__ S tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4)
    if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = x[(r0 + r) * ldx + c0 + tx];
  __syncthreads();
  for (int c = ty; c < 64; c += 4)
    if (c0 + c < cols && r0 + tx < rows) y[(c0 + c) * ldy + r0 + tx] = tile[tx][c];
}

// ---------------------------------------------------------------- embedding
template <typename T>
__global__ __launch_bounds__(kBlock) void embedding_fwd_kernel(const void* __restrict__ ids, int ids64,
                                                               const typename T::storage* __restrict__ w,
                                                               typename T::storage* __restrict__ y, int* bad,
                                                               int64_t n, int64_t vocab, int64_t h, int vec_ok) {
  constexpr int V = T::vec;
  const int64_t per = vec_ok ? h / V : h;
  const int64_t total = n * per;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / per, c = i % per;
    const int64_t id = ids64 ? ((const int64_t*)ids)[r] : (int64_t)((const int*)ids)[r];
    const bool ok = id >= 0 && id < vocab;
    if (!ok && c == 0 && bad) *bad = 1;
    if (vec_ok) {
      Vec<T> v;
      if (ok) {
        v = load_vec<T>(w + id * h + c * V);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) v.v[e] = 0.f;
      }
      store_vec<T>(y + r * h + c * V, v);
    } else {
      y[r * h + c] = ok ? w[id * h + c] : from_f32<T>(0.f);
    }
  }
}

Q3_DEV int64_t load_id(const void* ids, int ids64, int64_t i) {
  return ids64 ? ((const int64_t*)ids)[i] : (int64_t)((const int*)ids)[i];
}

// Stable counting rank: order[rank(i)] = i with positions sorted by (id, position).
__global__ __launch_bounds__(kBlock) void embedding_rank_kernel(const void* __restrict__ ids, int ids64,
                                                                int* __restrict__ order, int64_t n) {
  __shared__ int64_t chunk[kBlock];
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t mine = i < n ? load_id(ids, ids64, i) : 0;
  int64_t rank = 0;
  for (int64_t base = 0; base < n; base += kBlock) {
    __syncthreads();
    if (base + threadIdx.x < n) chunk[threadIdx.x] = load_id(ids, ids64, base + threadIdx.x);
    __syncthreads();
    const int64_t lim = n - base < kBlock ? n - base : kBlock;
    for (int64_t j = 0; j < lim; ++j) {
      const int64_t o = chunk[j];
      rank += (o < mine) || (o == mine && base + j < i);
    }
  }
  if (i < n) order[rank] = (int)i;
}

// One workgroup per sorted slot that starts a run of equal ids: sums the run's gradient rows in
// position order and writes the token's row of dw.
template <typename T>
__global__ __launch_bounds__(kBlock) void embedding_sum_kernel(const void* __restrict__ ids, int ids64,
                                                               const int* __restrict__ order,
                                                               const typename T::storage* __restrict__ dy,
                                                               typename T::storage* __restrict__ dw, int64_t n,
                                                               int64_t vocab, int64_t h) {
  const int64_t s = blockIdx.x;
  const int64_t id = load_id(ids, ids64, order[s]);
  if (id < 0 || id >= vocab) return;
  if (s > 0 && load_id(ids, ids64, order[s - 1]) == id) return;
  int64_t e = s + 1;
  while (e < n && load_id(ids, ids64, order[e]) == id) ++e;
  for (int64_t c = (int64_t)blockIdx.y * kBlock + threadIdx.x; c < h; c += (int64_t)gridDim.y * kBlock) {
    float acc = 0.f;
    for (int64_t k = s; k < e; ++k) acc += to_f32<T>(dy[(int64_t)order[k] * h + c]);
    dw[id * h + c] = from_f32<T>(acc);
  }
}

bool dtype_ok(int dt) { return dt == Q3_F32 || dt == Q3_F16 || dt == Q3_BF16; }

template <typename T> int swiglu_fwd_t(const void* g, const void* u, void* y, int64_t n, hipStream_t s) {
  typedef typename T::storage S;
  const int vec = aligned16<T>(g) && aligned16<T>(u) && aligned16<T>(y);
  swiglu_fwd_kernel<T><<<one_pass_grid(n / T::vec + 1), kBlock, 0, s>>>((const S*)g, (const S*)u, (S*)y, n,
                                                                                vec);
  return (int)hipGetLastError();
}
template <typename T>
int swiglu_bwd_t(const void* g, const void* u, const void* dy, void* dg, void* du, int64_t n, hipStream_t s) {
  typedef typename T::storage S;
  const int vec = aligned16<T>(g) && aligned16<T>(u) && aligned16<T>(dy) && aligned16<T>(dg) && aligned16<T>(du);
  swiglu_bwd_kernel<T><<<one_pass_grid(n / T::vec + 1), kBlock, 0, s>>>((const S*)g, (const S*)u,
                                                                                (const S*)dy, (S*)dg, (S*)du, n, vec);
  return (int)hipGetLastError();
}
template <typename T> int add_t(const void* a, const void* b, void* c, int64_t n, hipStream_t s) {
  typedef typename T::storage S;
  const int vec = aligned16<T>(a) && aligned16<T>(b) && aligned16<T>(c);
  add_kernel<T><<<q3_grid_for(n / T::vec + 1, kBlock), kBlock, 0, s>>>((const S*)a, (const S*)b, (S*)c, n, vec);
  return (int)hipGetLastError();
}
template <typename T> int fill_t(void* x, float v, int64_t n, hipStream_t s) {
  fill_kernel<T><<<q3_grid_for(n, kBlock), kBlock, 0, s>>>((typename T::storage*)x, v, n);
  return (int)hipGetLastError();
}
template <typename S, typename D> int cast_t2(const void* x, void* y, int64_t n, hipStream_t s) {
  cast_kernel<S, D><<<q3_grid_for(n, kBlock), kBlock, 0, s>>>((const typename S::storage*)x,
                                                               (typename D::storage*)y, n);
  return (int)hipGetLastError();
}
template <typename S> int cast_t(int dst, const void* x, void* y, int64_t n, hipStream_t s) {
  if (dst == Q3_BF16) return cast_t2<S, BF16>(x, y, n, s);
  if (dst == Q3_F16) return cast_t2<S, F16>(x, y, n, s);
  return cast_t2<S, F32>(x, y, n, s);
}
template <typename T>
int tables_t(const void* pos, int pos64, const float* f, void* c, void* sn, int64_t npos, int64_t d, hipStream_t s) {
  rope_tables_kernel<T><<<q3_grid_for(npos * (d / 2), kBlock), kBlock, 0, s>>>(
      pos, pos64, f, (typename T::storage*)c, (typename T::storage*)sn, npos, (int)(d / 2));
  return (int)hipGetLastError();
}
template <typename T>
int rope_t(const void* x, const void* c, const void* sn, void* y, int64_t b, int64_t seq, int64_t heads, int64_t d,
           int layout, int bwd, hipStream_t s) {
  typedef typename T::storage S;
  const int64_t rows = b * seq * heads;
  const bool vec = (d / 2) % T::vec == 0 && aligned16<T>(x) && aligned16<T>(c) && aligned16<T>(sn) &&
                   aligned16<T>(y);
  if (vec)
    rope_apply_vec_kernel<T><<<q3_grid_for(rows * (d / 2 / T::vec), kBlock), kBlock, 0, s>>>(
        (const S*)x, (const S*)c, (const S*)sn, (S*)y, rows, seq, heads, (int)d, layout, bwd);
  else
    rope_apply_scalar_kernel<T><<<q3_grid_for(rows * (d / 2), kBlock), kBlock, 0, s>>>(
        (const S*)x, (const S*)c, (const S*)sn, (S*)y, rows, seq, heads, (int)d, layout, bwd);
  return (int)hipGetLastError();
}
template <typename T>
int emb_fwd_t(const void* ids, int ids64, const void* w, void* y, int* bad, int64_t n, int64_t vocab, int64_t h,
              hipStream_t s) {
  typedef typename T::storage S;
  const int vec = h % T::vec == 0 && aligned16<T>(w) && aligned16<T>(y);
  const int64_t per = vec ? h / T::vec : h;
  embedding_fwd_kernel<T><<<q3_grid_for(n * per, kBlock), kBlock, 0, s>>>(ids, ids64, (const S*)w, (S*)y, bad, n,
                                                                           vocab, h, vec);
  return (int)hipGetLastError();
}
template <typename T>
int emb_bwd_t(const void* ids, int ids64, const void* dy, void* dw, int* order, int64_t n, int64_t vocab, int64_t h,
              hipStream_t s) {
  typedef typename T::storage S;
  fill_kernel<T><<<q3_grid_for(vocab * h, kBlock), kBlock, 0, s>>>((S*)dw, 0.f, vocab * h);
  embedding_rank_kernel<<<(unsigned)((n + kBlock - 1) / kBlock), kBlock, 0, s>>>(ids, ids64, order, n);
  int64_t gy = (h + kBlock - 1) / kBlock;
  if (gy > 16) gy = 16;
  embedding_sum_kernel<T><<<dim3((unsigned)n, (unsigned)gy), kBlock, 0, s>>>(ids, ids64, order, (const S*)dy, (S*)dw,
                                                                             n, vocab, h);
  return (int)hipGetLastError();
}

}  // namespace

#define Q3_DISPATCH(dt, FN, ...) \
  ((dt) == Q3_BF16 ? FN<BF16>(__VA_ARGS__) : (dt) == Q3_F16 ? FN<F16>(__VA_ARGS__) : FN<F32>(__VA_ARGS__))

extern "C" {

int q3_swiglu_fwd(int dtype, const void* g, const void* u, void* y, int64_t n, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && g && u && y && n > 0);
  return Q3_DISPATCH(dtype, swiglu_fwd_t, g, u, y, n, stream);
}

int q3_swiglu_bwd(int dtype, const void* g, const void* u, const void* dy, void* dg, void* du, int64_t n,
                  hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && g && u && dy && dg && du && n > 0);
  return Q3_DISPATCH(dtype, swiglu_bwd_t, g, u, dy, dg, du, n, stream);
}

int q3_swiglu_bwd_2d(int dtype, const void* g, int64_t ldg, const void* u, int64_t ldu, const void* dy, int64_t lddy,
                     void* dg, int64_t lddg, void* du, int64_t lddu, int64_t rows, int64_t cols, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && g && u && dy && dg && du && rows > 0 && cols > 0 && ldg >= cols && ldu >= cols &&
             lddy >= cols && lddg >= cols && lddu >= cols);
  const int64_t V = dtype == Q3_F32 ? 4 : 8;
  const bool vec = cols % V == 0 && ldg % V == 0 && ldu % V == 0 && lddy % V == 0 && lddg % V == 0 && lddu % V == 0 &&
                   aligned16<u16>(g) && aligned16<u16>(u) && aligned16<u16>(dy) && aligned16<u16>(dg) &&
                   aligned16<u16>(du) && rows * (cols / V) < (1ll << 31);
  const unsigned grid = vec ? one_pass_grid(rows * (cols / V)) : q3_grid_for(rows * cols, kBlock);
#define Q3_SWB2(T, S)                                                                                          \
  swiglu_bwd2d_kernel<T><<<grid, kBlock, 0, stream>>>((const S*)g, ldg, (const S*)u, ldu, (const S*)dy, lddy, \
                                                      (S*)dg, lddg, (S*)du, lddu, rows, cols, vec ? 1 : 0)
  if (dtype == Q3_BF16) Q3_SWB2(BF16, u16);
  else if (dtype == Q3_F16) Q3_SWB2(F16, u16);
  else Q3_SWB2(F32, float);
#undef Q3_SWB2
  return (int)hipGetLastError();
}

int q3_copy2d(int dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t cols,
              hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && y && rows > 0 && cols > 0 && ldx >= cols && ldy >= cols);
  const int64_t esz = dtype == Q3_F32 ? 4 : 2, V = 16 / esz;
  const bool vec = cols % V == 0 && ldx % V == 0 && ldy % V == 0 && aligned16<u16>(x) && aligned16<u16>(y);
  const unsigned grid = q3_grid_for(rows * (vec ? cols / V : cols), kBlock);
  if (esz == 4)
    copy2d_kernel<uint32_t><<<grid, kBlock, 0, stream>>>((const uint32_t*)x, ldx, (uint32_t*)y, ldy, rows, cols, vec);
  else
    copy2d_kernel<u16><<<grid, kBlock, 0, stream>>>((const u16*)x, ldx, (u16*)y, ldy, rows, cols, vec);
  return (int)hipGetLastError();
}

int q3_transpose2d(int dtype, const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows, int64_t cols,
                   hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && y && rows > 0 && cols > 0 && ldx >= cols && ldy >= rows &&
             (rows + 63) / 64 < 65536);
  if (dtype != Q3_F32 && cols % 128 == 0 && rows % 128 == 0 && ldx % 8 == 0 && ldy % 8 == 0 &&
      aligned16<u16>(x) && aligned16<u16>(y)) {
    dim3 g((unsigned)(cols / 128), (unsigned)(rows / 128));
    transpose2d16_lds_kernel<<<g, kBlock, 0, stream>>>((const u16*)x, ldx, (u16*)y, ldy, 0, 0);
    return (int)hipGetLastError();
  }
  if (dtype != Q3_F32 && cols % 8 == 0 && rows % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && aligned16<u16>(x) &&
      aligned16<u16>(y)) {
    dim3 g16((unsigned)((cols + 255) / 256), (unsigned)((rows + 63) / 64));
    transpose2d16_kernel<<<g16, kBlock, 0, stream>>>((const u16*)x, ldx, (u16*)y, ldy, rows, cols);
    return (int)hipGetLastError();
  }
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (dtype == Q3_F32)
    transpose2d_scalar_kernel<uint32_t><<<grid, kBlock, 0, stream>>>((const uint32_t*)x, ldx, (uint32_t*)y, ldy, rows,
                                                                     cols);
  else
    transpose2d_scalar_kernel<u16><<<grid, kBlock, 0, stream>>>((const u16*)x, ldx, (u16*)y, ldy, rows, cols);
  return (int)hipGetLastError();
}

int q3_add(int dtype, const void* a, const void* b, void* c, int64_t n, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && a && b && c && n > 0);
  return Q3_DISPATCH(dtype, add_t, a, b, c, n, stream);
}

int q3_cast(int src, int dst, const void* x, void* y, int64_t n, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(src) && dtype_ok(dst) && x && y && n > 0);
  return Q3_DISPATCH(src, cast_t, dst, x, y, n, stream);
}

int q3_fill(int dtype, void* x, float value, int64_t n, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && n > 0);
  return Q3_DISPATCH(dtype, fill_t, x, value, n, stream);
}

int q3_positions(int64_t* out, int64_t batch, int64_t seq, int64_t start, const int64_t* start_dev,
                 hipStream_t stream) {
  Q3_REQUIRE(out && batch > 0 && seq > 0 && start >= 0);
  positions_kernel<<<q3_grid_for(batch * seq, kBlock), kBlock, 0, stream>>>(out, batch * seq, seq, start, start_dev);
  return (int)hipGetLastError();
}

int q3_transpose(int dtype, const void* x, void* y, int64_t batch, int64_t rows, int64_t cols, int64_t ldy,
                 hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && y && batch > 0 && rows > 0 && cols > 0 && batch < 65536 && ldy >= rows);
  Q3_REQUIRE((ldy + 63) / 64 < 65536);
  if (dtype != Q3_F32 && ldy == rows && rows % 128 == 0 && cols % 128 == 0 && aligned16<u16>(x) &&
      aligned16<u16>(y)) {  // no padding rows to zero: whole 128 x 128 tiles through LDS
    dim3 g((unsigned)(cols / 128), (unsigned)(rows / 128), (unsigned)batch);
    transpose2d16_lds_kernel<<<g, kBlock, 0, stream>>>((const u16*)x, cols, (u16*)y, ldy, rows * cols, cols * ldy);
    return (int)hipGetLastError();
  }
  if (dtype != Q3_F32 && cols % 8 == 0 && ldy % 8 == 0 && aligned16<u16>(x) && aligned16<u16>(y)) {
    dim3 g16((unsigned)((cols + 255) / 256), (unsigned)((ldy + 63) / 64), (unsigned)batch);
    transpose16_kernel<<<g16, kBlock, 0, stream>>>((const u16*)x, (u16*)y, rows, cols, ldy);
    return (int)hipGetLastError();
  }
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((ldy + 63) / 64), (unsigned)batch);
  if (dtype == Q3_F32)
    transpose_kernel<uint32_t><<<grid, kBlock, 0, stream>>>((const uint32_t*)x, (uint32_t*)y, rows, cols, ldy);
  else
    transpose_kernel<u16><<<grid, kBlock, 0, stream>>>((const u16*)x, (u16*)y, rows, cols, ldy);
  return (int)hipGetLastError();
}

int q3_rope_tables(int dtype, const void* pos, int pos_is_int64, const float* inv_freq, void* cos, void* sin,
                   int64_t n_pos, int64_t d, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && pos && inv_freq && cos && sin && n_pos > 0 && d > 0 && d % 2 == 0);
  return Q3_DISPATCH(dtype, tables_t, pos, pos_is_int64, inv_freq, cos, sin, n_pos, d, stream);
}

int q3_rope_apply(int dtype, const void* x, const void* cos, const void* sin, void* y, int64_t batch, int64_t seq,
                  int64_t heads, int64_t d, int layout, int backward, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && x && cos && sin && y && batch > 0 && seq > 0 && heads > 0 && d > 0 && d % 2 == 0 &&
             (layout == 0 || layout == 1));
  return Q3_DISPATCH(dtype, rope_t, x, cos, sin, y, batch, seq, heads, d, layout, backward ? 1 : 0, stream);
}

int q3_embedding_fwd(int dtype, const void* ids, int ids_is_int64, const void* w, void* y, int* bad_ids,
                     int64_t n_ids, int64_t vocab, int64_t h, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && ids && w && y && n_ids > 0 && vocab > 0 && h > 0);
  return Q3_DISPATCH(dtype, emb_fwd_t, ids, ids_is_int64, w, y, bad_ids, n_ids, vocab, h, stream);
}

size_t q3_embedding_bwd_workspace_bytes(int64_t n_ids) { return (size_t)(n_ids > 0 ? n_ids : 1) * sizeof(int); }

int q3_embedding_bwd(int dtype, const void* ids, int ids_is_int64, const void* dy, void* dw, void* workspace,
                     int64_t n_ids, int64_t vocab, int64_t h, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && ids && dy && dw && workspace && n_ids > 0 && n_ids < (1ll << 31) && vocab > 0 &&
             h > 0 && n_ids < 65536ll * 32768ll);
  return Q3_DISPATCH(dtype, emb_bwd_t, ids, ids_is_int64, dy, dw, (int*)workspace, n_ids, vocab, h, stream);
}

}  // extern "C"

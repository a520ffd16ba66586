// Causal cross-entropy pieces: label shift, per-row online log-sum-exp over (a chunk of) the
// vocabulary, chunk merge + per-row loss, deterministic token mean, and the logits gradient.
//
// The same kernels serve the reference's CE on materialised [B,S,V] logits (one chunk = whole
// vocabulary) and the fused LM-head CE, where the logits of one vocabulary chunk at a time come
// from the matrix-core GEMM and are never materialised for the full vocabulary.
//
// Row r = (b, s) uses target tgt[r] = labels[b, s+1] for s < S-1 and ignore_index for s = S-1
// (the causal shift of kernels/loss.py:16-24); ignored rows contribute neither loss nor count.
#include "common.h"

namespace {

constexpr int kThreads = 256;

// (max, sum-exp) pair combine in base e.
Q3_DEV void lse_combine(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * __expf(m - mn) + s2 * __expf(m2 - mn);
  m = mn;
}

__global__ __launch_bounds__(kThreads) void shift_labels_kernel(const int64_t* __restrict__ labels,
                                                                int64_t* __restrict__ tgt, int64_t rows, int64_t seq,
                                                                int64_t ignore) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x; r < rows; r += stride)
    tgt[r] = (r % seq) < seq - 1 ? labels[r + 1] : ignore;
}

// One workgroup per row: m/s over z[r, 0:n] (row stride ld); picks z[r, tgt - col0] when the target
// falls inside [col0, col0 + n).
template <typename T>
__global__ __launch_bounds__(kThreads) void ce_stats_kernel(const typename T::storage* __restrict__ z, int64_t ld,
                                                            int64_t n, int64_t col0,
                                                            const int64_t* __restrict__ tgt,
                                                            float* __restrict__ m_out, float* __restrict__ s_out,
                                                            float* __restrict__ pick, int vec_ok) {
  constexpr int V = T::vec;
  __shared__ float rm[kThreads / 64], rs[kThreads / 64];
  const int64_t r = blockIdx.x;
  const typename T::storage* row = z + r * ld;
  float m = -INFINITY, s = 0.f;
  const int64_t nv = vec_ok ? n / V : 0;
  auto fold = [&](const Vec<T>& x) {
    float vm = x.v[0];
#pragma unroll
    for (int e = 1; e < V; ++e) vm = fmaxf(vm, x.v[e]);
    float vs = 0.f;
#pragma unroll
    for (int e = 0; e < V; ++e) vs += __expf(x.v[e] - vm);
    lse_combine(m, s, vm, vs);
  };
  int64_t i = threadIdx.x;
  for (; i + 3 * kThreads < nv; i += 4 * kThreads) {  // four 16-byte loads in flight
    Vec<T> x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = load_vec<T>(row + (i + u * kThreads) * V);
#pragma unroll
    for (int u = 0; u < 4; ++u) fold(x[u]);
  }
  for (; i < nv; i += kThreads) fold(load_vec<T>(row + i * V));
  for (int64_t i = nv * V + threadIdx.x; i < n; i += kThreads) lse_combine(m, s, to_f32<T>(row[i]), 1.f);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    lse_combine(m, s, m2, s2);
  }
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0) {
    rm[w] = m;
    rs[w] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = rm[0], S = rs[0];
    for (int i = 1; i < kThreads / 64; ++i) lse_combine(M, S, rm[i], rs[i]);
    m_out[r] = M;
    s_out[r] = S;
    const int64_t t = tgt[r];
    if (t >= col0 && t < col0 + n) pick[r] = to_f32<T>(row[t - col0]);
  }
}

// Merge the per-chunk (m, s) of each row (chunk-major arrays [nchunks][rows]), write lse and the
// per-row loss; flag targets outside [0, vocab) that are not ignore_index.  A workgroup takes
// kFinRows rows; thread t folds the partials c = t / kFinRows (mod kFinSlices) of row t % kFinRows,
// then the slices of each row merge in slice order (fixed partition and order: deterministic).
constexpr int kFinRows = 16, kFinSlices = kThreads / kFinRows;
__global__ __launch_bounds__(kThreads) void ce_finish_kernel(const float* __restrict__ m_part,
                                                             const float* __restrict__ s_part, int nchunks,
                                                             const float* __restrict__ pick,
                                                             const int64_t* __restrict__ tgt,
                                                             float* __restrict__ lse, float* __restrict__ loss_rows,
                                                             int* __restrict__ bad, int64_t rows, int64_t vocab,
                                                             int64_t ignore) {
  __shared__ float sm[kFinSlices][kFinRows], ss[kFinSlices][kFinRows];
  const int lr = threadIdx.x % kFinRows, sl = threadIdx.x / kFinRows;
  const int64_t r = (int64_t)blockIdx.x * kFinRows + lr;
  const int64_t rc = r < rows ? r : rows - 1;
  float m = -INFINITY, s = 0.f;
  int c = sl;
  for (; c + 3 * kFinSlices < nchunks; c += 4 * kFinSlices) {  // four partials in flight
    float pm[4], ps[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      pm[u] = m_part[(int64_t)(c + u * kFinSlices) * rows + rc];
      ps[u] = s_part[(int64_t)(c + u * kFinSlices) * rows + rc];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) lse_combine(m, s, pm[u], ps[u]);
  }
  for (; c < nchunks; c += kFinSlices) lse_combine(m, s, m_part[(int64_t)c * rows + rc], s_part[(int64_t)c * rows + rc]);
  sm[sl][lr] = m;
  ss[sl][lr] = s;
  __syncthreads();
  if (sl != 0 || r >= rows) return;
  m = sm[0][lr];
  s = ss[0][lr];
  for (int k = 1; k < kFinSlices; ++k) lse_combine(m, s, sm[k][lr], ss[k][lr]);
  const float l = m + __logf(s);
  lse[r] = l;
  const int64_t t = tgt[r];
  const bool valid = t != ignore && t >= 0 && t < vocab;
  if (t != ignore && !valid && bad) *bad = 1;
  loss_rows[r] = valid ? l - pick[r] : 0.f;
}

// loss = sum(loss_rows) / count(valid); one workgroup, fixed-order strided sums + fixed tree.
__global__ __launch_bounds__(kThreads) void ce_mean_kernel(const float* __restrict__ loss_rows,
                                                           const int64_t* __restrict__ tgt, int64_t rows,
                                                           int64_t vocab, int64_t ignore, float* __restrict__ loss,
                                                           float* __restrict__ count) {
  __shared__ float sl[kThreads], sc[kThreads];
  float a = 0.f, c = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += kThreads) {
    a += loss_rows[r];
    const int64_t t = tgt[r];
    c += (t != ignore && t >= 0 && t < vocab) ? 1.f : 0.f;
  }
  sl[threadIdx.x] = a;
  sc[threadIdx.x] = c;
  __syncthreads();
  for (int o = kThreads / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      sl[threadIdx.x] += sl[threadIdx.x + o];
      sc[threadIdx.x] += sc[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *loss = sl[0] / sc[0];
    *count = sc[0];
  }
}

// dz[r, c] = (exp(z[r, c] - lse[r]) - [c + col0 == tgt[r]]) * up / count for valid rows, else 0.
template <typename T, typename O>
__global__ __launch_bounds__(kThreads) void ce_grad_kernel(const typename T::storage* __restrict__ z, int64_t ld,
                                                           int64_t n, int64_t col0, const int64_t* __restrict__ tgt,
                                                           const float* __restrict__ lse,
                                                           const float* __restrict__ count,
                                                           const float* __restrict__ up,
                                                           typename O::storage* __restrict__ dz, int64_t ldo,
                                                           int64_t rows, int64_t vocab, int64_t ignore,
                                                           int vec_ok) {
  const int64_t r = blockIdx.x;
  const int64_t t = tgt[r];
  const bool valid = t != ignore && t >= 0 && t < vocab;
  const float scale = valid ? (up ? *up : 1.f) / *count : 0.f;
  const float l = lse[r];
  const typename T::storage* row = z + r * ld;
  typename O::storage* out = dz + r * ldo;
  // 8 columns per thread: 16-byte loads and stores (vec_ok: 16-byte aligned rows of both buffers)
  const int64_t n8 = vec_ok ? n / 8 : 0;
  for (int64_t i = (int64_t)blockIdx.y * kThreads + threadIdx.x; i < n8; i += (int64_t)gridDim.y * kThreads) {
    const int64_t c = i * 8;
    float zv[8];
    if constexpr (T::vec == 8) {
      const Vec<T> a = load_vec<T>(row + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) zv[e] = a.v[e];
    } else {
      const Vec<T> a = load_vec<T>(row + c), b = load_vec<T>(row + c + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        zv[e] = a.v[e];
        zv[4 + e] = b.v[e];
      }
    }
    float pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      pv[e] = valid ? (__expf(zv[e] - l) - ((c + e + col0 == t) ? 1.f : 0.f)) * scale : 0.f;
    if constexpr (O::vec == 8) {
      Vec<O> o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o.v[e] = pv[e];
      store_vec<O>(out + c, o);
    } else {
      Vec<O> o0, o1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o0.v[e] = pv[e];
        o1.v[e] = pv[4 + e];
      }
      store_vec<O>(out + c, o0);
      store_vec<O>(out + c + 4, o1);
    }
  }
  for (int64_t c = n8 * 8 + (int64_t)blockIdx.y * kThreads + threadIdx.x; c < n; c += (int64_t)gridDim.y * kThreads) {
    const float p = valid ? __expf(to_f32<T>(row[c]) - l) - ((c + col0 == t) ? 1.f : 0.f) : 0.f;
    out[c] = from_f32<O>(p * scale);
  }
}

bool dtype_ok(int dt) { return dt == Q3_F32 || dt == Q3_F16 || dt == Q3_BF16; }

template <typename T>
int stats_t(const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt, float* m, float* s, float* pick,
            int64_t rows, hipStream_t st) {
  typedef typename T::storage S;
  const int vec = ((uintptr_t)z % 16 == 0) && (ld % T::vec == 0);
  ce_stats_kernel<T><<<(unsigned)rows, kThreads, 0, st>>>((const S*)z, ld, n, col0, tgt, m, s, pick, vec);
  return (int)hipGetLastError();
}

template <typename T, typename O>
int grad_t2(const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt, const float* lse,
            const float* count, const float* up, void* dz, int64_t ldo, int64_t rows, int64_t vocab, int64_t ignore,
            hipStream_t st) {
  const int vec = ((uintptr_t)z % 16 == 0) && ((uintptr_t)dz % 16 == 0) && ld % 8 == 0 && ldo % 8 == 0;
  int64_t gx = (n + 8 * kThreads - 1) / (8 * kThreads);
  if (gx > 64) gx = 64;
  ce_grad_kernel<T, O><<<dim3((unsigned)rows, (unsigned)gx), kThreads, 0, st>>>(
      (const typename T::storage*)z, ld, n, col0, tgt, lse, count, up, (typename O::storage*)dz, ldo, rows, vocab,
      ignore, vec);
  return (int)hipGetLastError();
}

// dz (in the input's 16-bit type) and its transpose for one logits chunk: a workgroup takes 64 rows x
// 128 columns, computes dz with q3_ce_chunk_grad's expression, stores it row-major (16-byte stores; dz
// may be the logits buffer itself: every element is read before it is written by the same thread) and
// through an LDS tile (rows padded to 65 words: conflict-free row writes and column gathers) as
// dzt[col][row] with 16-byte stores of 8 rows.
template <typename T>
__global__ __launch_bounds__(kThreads) void ce_grad_t_kernel(const u16* z, int64_t ld, int64_t n, int64_t col0,
                                                             const int64_t* __restrict__ tgt,
                                                             const float* __restrict__ lse,
                                                             const float* __restrict__ count,
                                                             const float* __restrict__ up, u16* dz, int64_t ldo,
                                                             u16* __restrict__ dzt, int64_t lddzt, int64_t rows,
                                                             int64_t vocab, int64_t ignore) {
  constexpr int TR = 64, TC = 128, RP = TC + 2;
  __shared__ __attribute__((aligned(16))) u16 tile[TR * RP];
  const int64_t r0 = (int64_t)blockIdx.y * TR, c0 = (int64_t)blockIdx.x * TC;
  const int tid = threadIdx.x, ch = tid & 15, rr = tid >> 4;
  const int64_t col = c0 + 8 * ch;
  const bool colok = col < n;
  const float sc = (up ? *up : 1.f) / *count;
  i32x4 zv[4];
  int64_t tv[4];
  float lv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // every load first (clamped indices, masked below)
    const int64_t row = min(r0 + rr + 16 * k, rows - 1);
    zv[k] = *reinterpret_cast<const i32x4*>(z + row * ld + (colok ? col : 0));
    tv[k] = tgt[row];
    lv[k] = lse[row];
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t row = r0 + rr + 16 * k;
    const bool valid = tv[k] != ignore && tv[k] >= 0 && tv[k] < vocab;
    const Vec<T> a = unpack_vec<T>(zv[k]);
    Vec<T> o;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o.v[e] = valid ? (__expf(a.v[e] - lv[k]) - ((col + e + col0 == tv[k]) ? 1.f : 0.f)) * sc : 0.f;
    i32x4 pk;
#pragma unroll
    for (int w = 0; w < 4; ++w) pk[w] = (int)pack2<T>(o.v[2 * w], o.v[2 * w + 1]);
    if (row < rows && colok) *reinterpret_cast<i32x4*>(dz + row * ldo + col) = pk;
    uint32_t* tl = reinterpret_cast<uint32_t*>(tile + (rr + 16 * k) * RP + 8 * ch);
#pragma unroll
    for (int w = 0; w < 4; ++w) tl[w] = (uint32_t)pk[w];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // 8 lanes per output row: dzt[c0 + c][r0 + 8 q .. + 7]
    const int idx = tid + kThreads * k, q = idx & 7, c = idx >> 3;
    i32x4 v;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      v[w] = (int)((uint32_t)tile[(8 * q + 2 * w) * RP + c] | ((uint32_t)tile[(8 * q + 2 * w + 1) * RP + c] << 16));
    if (c0 + c < n && r0 + 8 * q < rows) *reinterpret_cast<i32x4*>(dzt + (c0 + c) * lddzt + r0 + 8 * q) = v;
  }
}

template <typename T>
int grad_t(int out_dtype, const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt, const float* lse,
           const float* count, const float* up, void* dz, int64_t ldo, int64_t rows, int64_t vocab, int64_t ignore,
           hipStream_t st) {
  if (out_dtype == Q3_BF16)
    return grad_t2<T, BF16>(z, ld, n, col0, tgt, lse, count, up, dz, ldo, rows, vocab, ignore, st);
  if (out_dtype == Q3_F16)
    return grad_t2<T, F16>(z, ld, n, col0, tgt, lse, count, up, dz, ldo, rows, vocab, ignore, st);
  return grad_t2<T, F32>(z, ld, n, col0, tgt, lse, count, up, dz, ldo, rows, vocab, ignore, st);
}

}  // namespace

extern "C" {

int q3_ce_shift_labels(const int64_t* labels, int64_t* tgt, int64_t batch, int64_t seq, int64_t ignore_index,
                       hipStream_t stream) {
  Q3_REQUIRE(labels && tgt && batch > 0 && seq > 0);
  shift_labels_kernel<<<q3_grid_for(batch * seq, kThreads), kThreads, 0, stream>>>(labels, tgt, batch * seq, seq,
                                                                                   ignore_index);
  return (int)hipGetLastError();
}

int q3_ce_chunk_stats(int dtype, const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt,
                      float* m_out, float* s_out, float* pick, int64_t rows, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && z && tgt && m_out && s_out && pick && n > 0 && rows > 0 && ld >= n &&
             rows < (1ll << 31));
  if (dtype == Q3_BF16) return stats_t<BF16>(z, ld, n, col0, tgt, m_out, s_out, pick, rows, stream);
  if (dtype == Q3_F16) return stats_t<F16>(z, ld, n, col0, tgt, m_out, s_out, pick, rows, stream);
  return stats_t<F32>(z, ld, n, col0, tgt, m_out, s_out, pick, rows, stream);
}

int q3_ce_finish(const float* m_part, const float* s_part, int nchunks, const float* pick, const int64_t* tgt,
                 float* lse, float* loss_rows, int* bad, float* loss, float* count, int64_t rows, int64_t vocab,
                 int64_t ignore_index, hipStream_t stream) {
  Q3_REQUIRE(m_part && s_part && nchunks > 0 && pick && tgt && lse && loss_rows && loss && count && rows > 0);
  ce_finish_kernel<<<(unsigned)((rows + kFinRows - 1) / kFinRows), kThreads, 0, stream>>>(
      m_part, s_part, nchunks, pick, tgt, lse, loss_rows, bad, rows, vocab, ignore_index);
  ce_mean_kernel<<<1, kThreads, 0, stream>>>(loss_rows, tgt, rows, vocab, ignore_index, loss, count);
  return (int)hipGetLastError();
}

int q3_ce_chunk_grad_t(int dtype, const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt,
                       const float* lse, const float* count, const float* up, void* dz, int64_t ldo, void* dzt,
                       int64_t lddzt, int64_t rows, int64_t vocab, int64_t ignore_index, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && z && tgt && lse && count && dz && dzt && n > 0 && rows > 0 &&
             rows < (1ll << 31) && n % 8 == 0 && rows % 8 == 0 && ld >= n && ldo >= n && lddzt >= rows &&
             ld % 8 == 0 && ldo % 8 == 0 && lddzt % 8 == 0 && (((uintptr_t)z | (uintptr_t)dz | (uintptr_t)dzt) & 15) == 0);
  // dz may be z itself (in place), but no other overlap
  Q3_REQUIRE(dz == z ? ldo == ld : true);
  const dim3 g((unsigned)((n + 127) / 128), (unsigned)((rows + 63) / 64));
  if (dtype == Q3_BF16)
    ce_grad_t_kernel<BF16><<<g, kThreads, 0, stream>>>((const u16*)z, ld, n, col0, tgt, lse, count, up, (u16*)dz, ldo,
                                                       (u16*)dzt, lddzt, rows, vocab, ignore_index);
  else
    ce_grad_t_kernel<F16><<<g, kThreads, 0, stream>>>((const u16*)z, ld, n, col0, tgt, lse, count, up, (u16*)dz, ldo,
                                                      (u16*)dzt, lddzt, rows, vocab, ignore_index);
  return (int)hipGetLastError();
}

int q3_ce_chunk_grad(int dtype, int out_dtype, const void* z, int64_t ld, int64_t n, int64_t col0, const int64_t* tgt,
                     const float* lse, const float* count, const float* up, void* dz, int64_t ldo, int64_t rows,
                     int64_t vocab, int64_t ignore_index, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && dtype_ok(out_dtype) && z && tgt && lse && count && dz && n > 0 && rows > 0 &&
             rows < (1ll << 31) && ld >= n && ldo >= n);
  if (dtype == Q3_BF16)
    return grad_t<BF16>(out_dtype, z, ld, n, col0, tgt, lse, count, up, dz, ldo, rows, vocab, ignore_index, stream);
  if (dtype == Q3_F16)
    return grad_t<F16>(out_dtype, z, ld, n, col0, tgt, lse, count, up, dz, ldo, rows, vocab, ignore_index, stream);
  return grad_t<F32>(out_dtype, z, ld, n, col0, tgt, lse, count, up, dz, ldo, rows, vocab, ignore_index, stream);
}

}  // extern "C"

// Single-GPU greedy decode: small-M GEMV, KV-cache append, split-KV decode attention and the
// greedy argmax/select step.  All four are bound by HBM traffic (weights, cache, logits).
#include "common.h"

namespace {

constexpr int kThreads = 256;

// ============================================================================ GEMV
// y[m, n] = sum_k x[m, k] * W[n, k] for M <= 8 rows of x.  A workgroup owns R consecutive rows of
// W and its 4 waves split K into interleaved 16-byte chunks (lane chunk c = wave*64 + lane +
// 256*i), so every weight byte is read once with fully coalesced 16-byte loads and each x chunk
// load is shared by R weight rows.  The R*M fp32 partials are reduced inside each wave (DPP /
// swizzle butterflies) and then across the 4 waves through LDS in a fixed order: deterministic.
template <typename T, int M, int R>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const u16* __restrict__ x, int64_t ldx,
                                                        const u16* __restrict__ W, u16* __restrict__ y, int64_t ldy,
                                                        int N, int K) {
  __shared__ float red[4][R * M];
  const int n0 = blockIdx.x * R;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = K / 8;
  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  for (int c = tid; c < nch; c += kThreads) {
    Vec<T> wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (n0 + r < N) {
        wv[r] = load_vec<T>(W + (int64_t)(n0 + r) * K + (int64_t)c * 8);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) wv[r].v[e] = 0.f;
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const Vec<T> xv = load_vec<T>(x + m * ldx + (int64_t)c * 8);
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][m] += wv[r].v[e] * xv.v[e];
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float s = group_sum<64>(acc[r][m]);
      if (lane == 0) red[wave][r * M + m] = s;
    }
  __syncthreads();
  if (tid < R * M) {
    const int r = tid / M, m = tid % M;
    if (n0 + r < N) {
      const float s = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
      y[m * ldy + n0 + r] = from_f32<T>(s);
    }
  }
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
// One wave per (b, query head, chunk of kChunk cached keys).  16 lanes own one key (8 of its 128
// dims each), so a wave scores 4 keys per step with 16-byte loads and a 16-lane DPP reduction; the
// chunk's scores sit in LDS for the max/exp pass; the V pass mirrors the K pass and the 4 key
// groups are folded at the end.  Writes the unnormalised partial output, its max and its sum.
constexpr int kChunk = 128;

template <typename T>
__global__ __launch_bounds__(64) void decode_attn_partial(const u16* __restrict__ q, int64_t qsb, int64_t qsh,
                                                          const u16* __restrict__ ck, const u16* __restrict__ cv,
                                                          int64_t ksb, int64_t ksh, float* __restrict__ opart,
                                                          float* __restrict__ mpart, float* __restrict__ lpart,
                                                          int Hq, int Hkv, int T_len, const int64_t* len_dev,
                                                          int capacity, int splits, float scale) {
  constexpr int D = 128;
  __shared__ float sc[kChunk];
  const int split = blockIdx.x, bh = blockIdx.y, b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hkv);
  const int lane = threadIdx.x, t = lane & 15, grp = lane >> 4;
  // len_dev holds the cache length before this token: the token itself is at that position.
  if (len_dev) T_len = min((int)*len_dev + 1, capacity);
  const int k0 = split * kChunk;
  const int kend = min(T_len, k0 + kChunk);
  const int64_t pi0 = (int64_t)bh * splits + split;
  if (k0 >= T_len) {  // split beyond the live length (fixed-size launch): an empty partial
    for (int e = lane; e < D; e += 64) opart[pi0 * D + e] = 0.f;
    if (lane == 0) {
      mpart[pi0] = -INFINITY;
      lpart[pi0] = 0.f;
    }
    return;
  }
  const u16* kb = ck + b * ksb + hk * ksh;
  const u16* vb = cv + b * ksb + hk * ksh;
  const Vec<T> qv = load_vec<T>(q + b * qsb + h * qsh + t * 8);
  for (int it = 0; it < kChunk / 4; ++it) {
    const int j = it * 4 + grp, key = k0 + j;
    float s = 0.f;
    if (key < kend) {
      const Vec<T> kv = load_vec<T>(kb + (int64_t)key * D + t * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += qv.v[e] * kv.v[e];
    }
    s = group_sum<16>(s);
    if (t == 0) sc[j] = key < kend ? s * scale : -INFINITY;
  }
  __syncthreads();
  float m = fmaxf(sc[lane], sc[lane + 64]);
  m = group_max<64>(m);
  const float p0 = __expf(sc[lane] - m), p1 = __expf(sc[lane + 64] - m);
  const float l = group_sum<64>(p0 + p1);
  __syncthreads();
  sc[lane] = p0;
  sc[lane + 64] = p1;
  __syncthreads();
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < kChunk / 4; ++it) {
    const int j = it * 4 + grp, key = k0 + j;
    if (key < kend) {
      const float p = sc[j];
      const Vec<T> vv = load_vec<T>(vb + (int64_t)key * D + t * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += p * vv.v[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] += __shfl_xor(o[e], 16, 64);
    o[e] += __shfl_xor(o[e], 32, 64);
  }
  const int64_t pi = (int64_t)bh * splits + split;
  if (grp == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) opart[pi * D + t * 8 + e] = o[e];
  }
  if (lane == 0) {
    mpart[pi] = m;
    lpart[pi] = l;
  }
}

// out[b, h, :] = sum_j exp(m_j - M) o_j / sum_j exp(m_j - M) l_j over the splits (fixed order).
template <typename T>
__global__ __launch_bounds__(64) void decode_attn_merge(const float* __restrict__ opart,
                                                        const float* __restrict__ mpart,
                                                        const float* __restrict__ lpart, u16* __restrict__ out,
                                                        int64_t osb, int64_t osh, int Hq, int splits) {
  constexpr int D = 128;
  const int bh = blockIdx.x, b = bh / Hq, h = bh % Hq, lane = threadIdx.x;
  float M = -INFINITY;
  for (int j = 0; j < splits; ++j) M = fmaxf(M, mpart[(int64_t)bh * splits + j]);
  float den = 0.f, o0 = 0.f, o1 = 0.f;
  for (int j = 0; j < splits; ++j) {
    const int64_t pi = (int64_t)bh * splits + j;
    if (mpart[pi] == -INFINITY) continue;  // empty split
    const float w = __expf(mpart[pi] - M);
    den += w * lpart[pi];
    o0 += w * opart[pi * D + lane];
    o1 += w * opart[pi * D + 64 + lane];
  }
  u16* orow = out + b * osb + h * osh;
  orow[lane] = from_f32<T>(o0 / den);
  orow[64 + lane] = from_f32<T>(o1 / den);
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

template <typename T, int M, int R>
int gemv_launch(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t n, int64_t k,
                hipStream_t s) {
  gemv_kernel<T, M, R><<<(unsigned)((n + R - 1) / R), kThreads, 0, s>>>((const u16*)x, ldx, (const u16*)w, (u16*)y,
                                                                         ldy, (int)n, (int)k);
  return (int)hipGetLastError();
}

template <typename T, int M>
int gemv_r(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t n, int64_t k, hipStream_t s) {
  // Enough workgroups to keep every CU streaming: fewer rows per workgroup for narrow outputs.
  if (n >= 8192) return gemv_launch<T, M, 4>(x, ldx, w, y, ldy, n, k, s);
  if (n >= 4096) return gemv_launch<T, M, 2>(x, ldx, w, y, ldy, n, k, s);
  return gemv_launch<T, M, 1>(x, ldx, w, y, ldy, n, k, s);
}

template <typename T>
int gemv_m(int m, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t n, int64_t k,
           hipStream_t s) {
  switch (m) {
    case 1: return gemv_r<T, 1>(x, ldx, w, y, ldy, n, k, s);
    case 2: return gemv_r<T, 2>(x, ldx, w, y, ldy, n, k, s);
    case 3: return gemv_r<T, 3>(x, ldx, w, y, ldy, n, k, s);
    case 4: return gemv_r<T, 4>(x, ldx, w, y, ldy, n, k, s);
    case 5: return gemv_r<T, 5>(x, ldx, w, y, ldy, n, k, s);
    case 6: return gemv_r<T, 6>(x, ldx, w, y, ldy, n, k, s);
    case 7: return gemv_r<T, 7>(x, ldx, w, y, ldy, n, k, s);
    default: return gemv_r<T, 8>(x, ldx, w, y, ldy, n, k, s);
  }
}

}  // namespace

extern "C" {

int q3_gemv(int dtype, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t m, int64_t n,
            int64_t k, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && x && w && y && m >= 1 && m <= 8 && n > 0 && k > 0);
  Q3_REQUIRE(k % 8 == 0 && ldx % 8 == 0 && ldx >= k && ldy >= n && al16(x) && al16(w) && n < (1ll << 31));
  if (dtype == Q3_BF16) return gemv_m<BF16>((int)m, x, ldx, w, y, ldy, n, k, stream);
  return gemv_m<F16>((int)m, x, ldx, w, y, ldy, n, k, stream);
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

size_t q3_decode_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t T_len) {
  const int64_t splits = (T_len + kChunk - 1) / kChunk;
  return (size_t)(B * Hq * splits) * (128 + 2) * sizeof(float);
}

int q3_decode_attention(int dtype, const void* q, int64_t qsb, int64_t qsh, const void* cache_k, const void* cache_v,
                        int64_t ksb, int64_t ksh, void* out, int64_t osb, int64_t osh, void* workspace, int64_t B,
                        int64_t Hq, int64_t Hkv, int64_t T_len, const int64_t* len_dev, int64_t capacity, int64_t D,
                        float scale, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && q && cache_k && cache_v && out && workspace && B > 0 &&
             Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && T_len > 0 && T_len <= capacity && D == 128 && B * Hq < 65536);
  // A device-resident length launches the fixed split count of the whole capacity (graph replay).
  const int64_t splits = ((len_dev ? capacity : T_len) + kChunk - 1) / kChunk;
  float* opart = (float*)workspace;
  float* mpart = opart + B * Hq * splits * 128;
  float* lpart = mpart + B * Hq * splits;
  dim3 grid((unsigned)splits, (unsigned)(B * Hq));
  if (dtype == Q3_BF16) {
    decode_attn_partial<BF16><<<grid, 64, 0, stream>>>((const u16*)q, qsb, qsh, (const u16*)cache_k,
                                                       (const u16*)cache_v, ksb, ksh, opart, mpart, lpart, (int)Hq,
                                                       (int)Hkv, (int)T_len, len_dev, (int)capacity, (int)splits, scale);
    decode_attn_merge<BF16><<<(unsigned)(B * Hq), 64, 0, stream>>>(opart, mpart, lpart, (u16*)out, osb, osh, (int)Hq,
                                                                   (int)splits);
  } else {
    decode_attn_partial<F16><<<grid, 64, 0, stream>>>((const u16*)q, qsb, qsh, (const u16*)cache_k,
                                                      (const u16*)cache_v, ksb, ksh, opart, mpart, lpart, (int)Hq,
                                                      (int)Hkv, (int)T_len, len_dev, (int)capacity, (int)splits, scale);
    decode_attn_merge<F16><<<(unsigned)(B * Hq), 64, 0, stream>>>(opart, mpart, lpart, (u16*)out, osb, osh, (int)Hq,
                                                                  (int)splits);
  }
  return (int)hipGetLastError();
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

// Causal GQA flash attention, forward and backward.
//
// Layouts: Q/O/dO/dQ [B,Hq,Lq,D], K/V/dK/dV [B,Hkv,Lk,D] (row-major, D contiguous); query head h
// reads KV head h / (Hq/Hkv).  Causal with a suffix offset: query i sees keys j <= i + (Lk - Lq).
// LSE [B,Hq,Lq] is the natural-log row logsumexp of the scaled scores; softmax runs in base 2 on
// scores pre-multiplied by scale*log2(e).
//
// Matrix-core path (bf16/fp16, D in {32, 64, 128}): every contraction is a v_mfma_f32_32x32x16.
// An MFMA operand must have its contraction index contiguous per lane, so operands contracted
// over the sequence axis (V in P.V; K in dS.K; Q, dO in dK/dV) are supplied by the host as
// sequence-contiguous transposed copies (Vt, Kt, Qt, dOt: [.., D, Lpad], Lpad = L rounded up to 8,
// zero padded), made by the transpose kernel.  Score tiles are computed transposed
// (S^T = K Q^T), so a lane owns one query and holds 32 key scores in registers: the softmax max/sum
// is an in-lane reduction plus one cross-half swizzle, and the probabilities are already laid out
// as the B operand of the next MFMA (with a fixed permutation of the 16 keys of each k-step that
// the A operand reads mirror).
//
// SIMT path: one wave per query (forward, dQ) or per key (dK/dV) with fp32 math; used for fp32
// and other head sizes.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <typename T> Q3_DEV f32x16 mma(bf16x8_t a, bf16x8_t b, f32x16 c);
template <> Q3_DEV f32x16 mma<BF16>(bf16x8_t a, bf16x8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <> Q3_DEV f32x16 mma<F16>(bf16x8_t a, bf16x8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                 0, 0);
}

template <typename T> Q3_DEV f32x4 mma16(bf16x8_t a, bf16x8_t b, f32x4 c) { return mfma_16x16x32<T>(a, b, c); }

Q3_DEV f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}
Q3_DEV i32x4 ld16(const u16* p) { return *reinterpret_cast<const i32x4*>(p); }
Q3_DEV bf16x8_t as_frag(i32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// Pack 8 accumulator values (v0..v0+7 of one 32x32 tile) into a B-operand fragment.
template <typename T> Q3_DEV bf16x8_t pack8(const f32x16& a, int v0) {
  i32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (int)pack2<T>(a[v0 + 2 * i], a[v0 + 2 * i + 1]);
  return as_frag(r);
}

// Row (key/query) index inside a 32x32 accumulator tile for element v of lane `lane`.
Q3_DEV int acc_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// Element strides (batch, head, position) of a [B, H, L, D] operand whose D axis is contiguous.
struct Lay {
  int64_t b, h, s;
};

// ============================================================================ forward (MFMA)
// Workgroup: 4 waves x 32 queries of one (b, h); each lane owns one query (scores are computed
// transposed, S^T = K Q^T) and walks key tiles of 64 with an online softmax.  K and V^T tiles go
// global -> LDS with wave-wide global_load_lds_dwordx4 into a 2-stage ring (no register staging, so two 4-wave
// workgroups fit per CU); LDS rows are unpadded and XOR-swizzled by 16-byte chunk so every MFMA
// operand read is bank-conflict free.  Tiles entirely below the causal diagonal skip the mask, and
// the output rescale is skipped when no lane's running max moved.
// Ring-buffer wait: let the tile that is about to be read land while up to `younger` later tiles of
// PER loads each stay in flight (vmcnt(younger * PER)), then a workgroup barrier that waits only for
// LDS reads -- __syncthreads()' release fence would drain every in-flight tile (vmcnt(0)).
template <int PER> Q3_DEV void ring_wait(int younger) {
  switch (younger) {
    case 0: __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8)); break;
    case 1: __builtin_amdgcn_s_waitcnt(((PER) & 15) | (((PER) >> 4) << 14) | (7 << 4) | (0 << 8)); break;
    case 2: __builtin_amdgcn_s_waitcnt(((2 * PER) & 15) | (((2 * PER) >> 4) << 14) | (7 << 4) | (0 << 8)); break;
    default: __builtin_amdgcn_s_waitcnt(((3 * PER) & 15) | (((3 * PER) >> 4) << 14) | (7 << 4) | (0 << 8)); break;
  }
  static_assert(3 * PER < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS destination pointer of a direct-to-LDS load
typedef __attribute__((address_space(3))) void* lds_vp;

template <int CPR> Q3_DEV int chunk_swz(int r) {
  if constexpr (CPR == 16) return r & 15;
  else if constexpr (CPR == 8) return (r ^ (r >> 3)) & 7;
  else return ((r >> 2) ^ (r >> 5)) & 3;
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_v2(const u16* __restrict__ Q, Lay ql, const u16* __restrict__ K,
                                                        Lay kl, const u16* __restrict__ Vt, u16* __restrict__ O,
                                                        float* __restrict__ LSE, int Hq, int Hkv, int Lq, int Lk,
                                                        int ldvt, float scale2) {
  constexpr int BN = 64, KS = D / 16, DT = D / 32;
  constexpr int CPK = D / 8, RPK = 64 / CPK;      // K: 16-byte chunks per row, rows per wave load
  constexpr int CPV = BN / 8, RPV = 64 / CPV;     // V^T rows (one d each) of BN keys
  constexpr int KLOADS = BN / RPK, VLOADS = D / RPV;
  constexpr int LPW = (KLOADS + VLOADS) / 4;      // wave loads per tile (4 waves)
  static_assert((KLOADS + VLOADS) % 4 == 0, "loads split over 4 waves");
  constexpr int KBYTES = BN * D * 2, STAGE = KBYTES + D * BN * 2;
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE];

  const int nqt = (Lq + 127) / 128;
  const int qt = nqt - 1 - (int)blockIdx.x;
  const int bh = blockIdx.y, b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hkv);
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int off = Lk - Lq;
  const int q0 = qt * 128 + wave * 32;
  const int qi = q0 + (lane & 31);
  const u16* Qb = Q + b * ql.b + h * ql.h;
  const u16* Kb = K + b * kl.b + hk * kl.h;
  const u16* Vb = Vt + (int64_t)(b * Hkv + hk) * D * ldvt;

  bf16x8_t qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qf[ks] = qi < Lq ? as_frag(ld16(Qb + qi * ql.s + ks * 16 + g * 8)) : as_frag(i32x4{0, 0, 0, 0});

  const int qlast_blk = min(qt * 128 + 127, Lq - 1) + off;
  const int ntiles = (min(Lk, qlast_blk + 1) + BN - 1) / BN;
  const int qfirst_wave = q0 + off;
  const int qlast_wave = min(q0 + 31, Lq - 1) + off;
  const int qpos = qi + off;

  // wave load i of a tile: global row/chunk of this lane and its LDS destination offset
  auto issue = [&](int stage, int t) {
    const int k0 = t * BN;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int w = wave + 4 * i;
      const void* src;
      int dst;
      if (w < KLOADS) {
        const int r = w * RPK + lane / CPK;
        const int c = (lane % CPK) ^ chunk_swz<CPK>(r);
        src = Kb + (int64_t)min(k0 + r, Lk - 1) * kl.s + c * 8;
        dst = stage * STAGE + w * RPK * D * 2;
      } else {
        const int r = (w - KLOADS) * RPV + lane / CPV;   // d
        const int c = (lane % CPV) ^ chunk_swz<CPV>(r);
        src = Vb + (int64_t)r * ldvt + min(k0 + c * 8, ldvt - 8);
        dst = stage * STAGE + KBYTES + (w - KLOADS) * RPV * BN * 2;
      }
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds + dst), 16, 0, 0);
    }
  };

  float m = -INFINITY, l = 0.f;
  f32x16 oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) oacc[i] = zero16();
  const int kr = lane & 31;
  const int kswz = chunk_swz<CPK>(kr), kswz2 = chunk_swz<CPK>(kr + 32);

  if (ntiles > 0) issue(0, 0);
  for (int t = 0; t < ntiles; ++t) {
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));  // vmcnt(0)
    __syncthreads();
    if (t + 1 < ntiles) issue((t + 1) & 1, t + 1);
    const int k0 = t * BN;
    if (k0 > qlast_wave) continue;
    const char* kbase = lds + (t & 1) * STAGE;
    const char* vbase = kbase + KBYTES;
    f32x16 sacc[2] = {zero16(), zero16()};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = ks * 2 + g;
      sacc[0] = mma<T>(as_frag(*reinterpret_cast<const i32x4*>(kbase + kr * D * 2 + ((c ^ kswz) << 4))), qf[ks], sacc[0]);
      sacc[1] = mma<T>(as_frag(*reinterpret_cast<const i32x4*>(kbase + (kr + 32) * D * 2 + ((c ^ kswz2) << 4))), qf[ks],
                       sacc[1]);
    }
    float mx = -INFINITY;
    if (k0 + BN - 1 <= qfirst_wave) {  // whole tile visible to every query of the wave
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          sacc[tt][v] *= scale2;
          mx = fmaxf(mx, sacc[tt][v]);
        }
    } else {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + tt * 32 + acc_row(v, lane);
          const float sv = key <= qpos ? sacc[tt][v] * scale2 : -INFINITY;
          sacc[tt][v] = sv;
          mx = fmaxf(mx, sv);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx);
    const float muse = mnew == -INFINITY ? 0.f : mnew;
    float ps = 0.f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = __builtin_amdgcn_exp2f(sacc[tt][v] - muse);
        sacc[tt][v] = p;
        ps += p;
      }
    ps += __shfl_xor(ps, 32, 64);
    if (__any(mnew != m)) {
      const float alpha = __builtin_amdgcn_exp2f(m - muse);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) oacc[dt][v] *= alpha;
    }
    l += ps;
    m = mnew;
#pragma unroll
    for (int c = 0; c < BN / 16; ++c) {
      const bf16x8_t pb = pack8<T>(sacc[c >> 1], (c & 1) * 8);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int r = dt * 32 + (lane & 31);
        const char* row = vbase + r * BN * 2;
        // keys {16c + 4g .. +3, 16c + 8 + 4g .. +3}: one 16-byte chunk of the permuted V^T row
        const i32x4 v4 = *reinterpret_cast<const i32x4*>(row + (((2 * c + g) ^ chunk_swz<CPV>(r)) << 4));
        oacc[dt] = mma<T>(as_frag(v4), pb, oacc[dt]);
      }
    }
  }

  if (qi < Lq) {
    const float inv = 1.f / l;
    u16* orow = O + b * ql.b + h * ql.h + qi * ql.s;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int d = dt * 32 + 8 * vg + 4 * g;
        typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
        i32x2 w;
        w[0] = (int)pack2<T>(oacc[dt][4 * vg] * inv, oacc[dt][4 * vg + 1] * inv);
        w[1] = (int)pack2<T>(oacc[dt][4 * vg + 2] * inv, oacc[dt][4 * vg + 3] * inv);
        *reinterpret_cast<i32x2*>(orow + d) = w;
      }
    if (g == 0) LSE[(int64_t)bh * Lq + qi] = (m + __log2f(l)) * kLn2;
  }
}

// ============================================================================ forward, D = 128 (MFMA 16x16x32)
// Workgroup: 8 waves sharing one KV head: wave w serves query head hk*GRP + (w % GH) (GH heads of
// the GQA group per workgroup) and 32 query positions q0 .. q0+31 (8/GH position groups), so every
// K/V tile in LDS feeds 256 query rows.  Scores are computed transposed, S^T = K Q^T, in 16x16
// tiles: lane (G = lane/16, r16 = lane%16) owns queries q0 + r16 and q0 + 16 + r16 and holds 4 keys
// of each 16-key tile.  Which K row feeds MFMA row r is chosen so that the two tiles of a 32-key
// step hand over P in exactly the key order of a 16-byte chunk of the permuted V^T copy
// (positions 0-3, 8-11, 4-7, 12-15 of every 16-block): P is the B operand of P.V as it comes out
// of the exponentials.  Row statistics need one max over the 4 lanes of a query (gfx950
// permlane16/32 swaps); the row sums come from the matrix cores (a block of ones times P, beside
// P.V), so the VALU forms no sums.
// Online softmax with a lazy rescale: the running max m (raw score units) moves only when a block
// max exceeds it by more than 8 / scale2 (a factor 2^8 in p), so O is rarely rescaled; p <= 2^8
// is exact in fp32 and in the bf16/fp16 P operand range.
// Pipeline per 64-key block j: P(j-1).V(j-1) and S(j+1) = K(j+1).Q^T run on the matrix cores while
// softmax(S(j)) runs on the VALU; steady-state blocks (unmasked, both neighbours present) are one
// basic block of 8 fenced steps, each with 8 MFMAs, the next step's 4 operand fragments and one
// part of the softmax.  K and V^T tiles go global -> LDS with direct-to-LDS loads into 2-stage
// rings, issued one block ahead.
Q3_DEV float xmax4(float x) {  // max over lanes {l, l^16, l^32, l^48}
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __builtin_fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
// LDS swizzles (16-byte chunk index XOR): K rows (16 chunks) by rows {0-7, 16-23} / {8-15, 24-31}
// of each 32-row group, V^T rows (8 chunks) by row pair.
Q3_DEV int kswz3(int r) { return (r & 7) | (((r >> 4) & 1) << 3); }
Q3_DEV int vswz3(int r) { return (r >> 1) & 7; }

template <typename T, int GH, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_v3(
    const u16* __restrict__ Q, Lay ql, const u16* __restrict__ K, Lay kl, const u16* __restrict__ Vt,
    u16* __restrict__ O, float* __restrict__ LSE, int Hq, int Hkv, int Lq, int Lk, int ldvt, float scale2) {
  constexpr int D = 128, BN = 64, QT = 32 * (NW / GH);
  constexpr int KST = BN * D * 2, VST = D * BN * 2;
  __shared__ __attribute__((aligned(1024))) char lds[2 * KST + 2 * VST];
  char* const kring = lds;
  char* const vring = lds + 2 * KST;

  const int nqt = (Lq + QT - 1) / QT;
  const int qt = nqt - 1 - (int)blockIdx.y;  // longest query tiles first
  const int tid = threadIdx.x, lane = tid & 63, G = lane >> 4, r16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int HB = Hq / GH, b = (int)blockIdx.x / HB, h = ((int)blockIdx.x % HB) * GH + wave % GH;
  const int hk = h / (Hq / Hkv), bh = b * Hq + h;
  const int off = Lk - Lq;
  const int q0 = qt * QT + (wave / GH) * 32;
  const u16* Qb = Q + b * ql.b + h * ql.h;
  const u16* Kb = K + b * kl.b + hk * kl.h;
  const u16* Vb = Vt + (int64_t)(b * Hkv + hk) * D * ldvt;

  bf16x8_t qf[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[u][ks] = as_frag(ld16(Qb + (int64_t)min(q0 + 16 * u + r16, Lq - 1) * ql.s + 32 * ks + 8 * G));

  const int nb = (min(Lk, min(qt * QT + QT - 1, Lq - 1) + off + 1) + BN - 1) / BN;  // workgroup blocks
  const int nbw = min(nb, (min(Lk, min(q0 + 31, Lq - 1) + off + 1) + BN - 1) / BN);  // this wave's
  const int qfirst_w = q0 + off;
  const int nfull = min(nbw, max(0, (qfirst_w + 1) / BN));  // blocks fully visible to the wave
  const int qpos[2] = {q0 + r16 + off, q0 + 16 + r16 + off};

  auto issueK = [&](int j) {  // 16 wave loads of 4 rows x 256 B, 2 per wave
    const int k0 = j * BN;
    char* base = kring + (j & 1) * KST;
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i) {
      const int w = wave + NW * i;
      const int r = w * 4 + (lane >> 4);
      const int c = (lane & 15) ^ kswz3(r);
      const u16* src = Kb + (int64_t)min(k0 + r, Lk - 1) * kl.s + c * 8;
      __builtin_amdgcn_global_load_lds(src, (lds_vp)(base + w * 1024), 16, 0, 0);
    }
  };
  auto issueV = [&](int j) {  // 16 wave loads of 8 V^T rows x 128 B, 2 per wave
    const int k0 = j * BN;
    char* base = vring + (j & 1) * VST;
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i) {
      const int w = wave + NW * i;
      const int r = w * 8 + (lane >> 3);
      const int c = (lane & 7) ^ vswz3(r);
      const u16* src = Vb + (int64_t)r * ldvt + min(k0 + c * 8, ldvt - 8);
      __builtin_amdgcn_global_load_lds(src, (lds_vp)(base + w * 1024), 16, 0, 0);
    }
  };

  // MFMA row r16 of key tile kt reads K row 32 (kt/2) + 8 (kt%2) + krow0 with
  // krow0 = 4 ((r16/4) % 2) + 16 (r16/8) + r16 % 4; element i of that tile on lane group G is then
  // key 32 (kt/2) + 8 (kt%2) + kbase + i, kbase = 4 (G % 2) + 16 (G / 2).  The K swizzle of every
  // such row is r16, so one LDS offset per k-step; tile and stage offsets are immediates.
  const int krow0 = 4 * ((r16 >> 2) & 1) + 16 * (r16 >> 3) + (r16 & 3);
  const int kbase = 4 * (G & 1) + 16 * (G >> 1);
  int koff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = krow0 * 256 + (((4 * ks + G) ^ r16) << 4);
  int voff[2];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) voff[kc] = r16 * 128 + (((4 * kc + G) ^ vswz3(r16)) << 4);
  constexpr int ktoff[4] = {0, 8 * 256, 32 * 256, 40 * 256};

  f32x4 S[4][2];
  i32x4 P[2][2];
  f32x4 oacc[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int u = 0; u < 2; ++u) oacc[dt][u] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Row sums on the matrix cores: a block of ones as the A operand gives lsum[u] = sum over keys of P,
  // every element of the quad equal (the P that P.V uses, rescaled with O like a 129th column).
  const uint32_t one2 = pack2<T>(1.f, 1.f);
  const i32x4 ones = i32x4{(int)one2, (int)one2, (int)one2, (int)one2};
  f32x4 lsum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  float m[2] = {-INFINITY, -INFINITY}, alpha[2] = {1.f, 1.f};
  bool pend = false;
  const float thr = 8.f / scale2;

  auto qk = [&](int j) {
    const char* kb = kring + (j & 1) * KST;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(kb + koff[ks] + ktoff[kt]);
#pragma unroll
        for (int u = 0; u < 2; ++u)
          S[kt][u] = mma16<T>(as_frag(a), qf[u][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : S[kt][u]);
      }
  };
  auto pv = [&](int j) {
    const char* vb = vring + (j & 1) * VST;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(vb + voff[kc] + dt * 16 * 128);
#pragma unroll
        for (int u = 0; u < 2; ++u) oacc[dt][u] = mma16<T>(as_frag(a), as_frag(P[u][kc]), oacc[dt][u]);
      }
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int u = 0; u < 2; ++u) lsum[u] = mma16<T>(as_frag(ones), as_frag(P[u][kc]), lsum[u]);
  };
  auto rescale = [&]() {
    if (pend) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) oacc[dt][u][i] *= alpha[u];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) lsum[u][i] *= alpha[u];
    }
  };
  // row max of S(j) for query tile u, then (after both) the lazy-rescale decision
  auto rowmax = [&](int u) {
    float x = __builtin_fmaxf(__builtin_fmaxf(S[0][u][0], S[0][u][1]), __builtin_fmaxf(S[0][u][2], S[0][u][3]));
#pragma unroll
    for (int kt = 1; kt < 4; ++kt)
      x = __builtin_fmaxf(__builtin_fmaxf(x, __builtin_fmaxf(S[kt][u][0], S[kt][u][1])),
                          __builtin_fmaxf(S[kt][u][2], S[kt][u][3]));
    return xmax4(x);
  };
  float ms[2];
  auto decide = [&](const float (&bm)[2]) {
    bool need[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      need[u] = bm[u] > m[u] + thr;
      const float mn = need[u] ? bm[u] : m[u];
      alpha[u] = __builtin_amdgcn_exp2f((m[u] - mn) * scale2);
      m[u] = mn;
      ms[u] = mn == -INFINITY ? 0.f : mn * scale2;
    }
    pend = __any(need[0] || need[1]);
  };
  auto expo = [&](int u, int kt) {  // p = exp2(s * scale2 - m * scale2)
#pragma unroll
    for (int i = 0; i < 4; ++i) S[kt][u][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[kt][u][i], scale2, -ms[u]));
  };
  auto pack = [&]() {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        i32x4 w;
        w[0] = (int)pack2<T>(S[2 * c][u][0], S[2 * c][u][1]);
        w[1] = (int)pack2<T>(S[2 * c][u][2], S[2 * c][u][3]);
        w[2] = (int)pack2<T>(S[2 * c + 1][u][0], S[2 * c + 1][u][1]);
        w[3] = (int)pack2<T>(S[2 * c + 1][u][2], S[2 * c + 1][u][3]);
        P[u][c] = w;
      }
  };
  auto softmax = [&](int j, bool mask) {
    if (mask) {
      const int qrel[2] = {qpos[0] - j * BN - kbase, qpos[1] - j * BN - kbase};
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            S[kt][u][i] = 32 * (kt >> 1) + 8 * (kt & 1) + i <= qrel[u] ? S[kt][u][i] : -INFINITY;
    }
    const float bm[2] = {rowmax(0), rowmax(1)};
    decide(bm);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) expo(u, kt);
    pack();
  };
  // Steady state: steps 0-3 P(j-1).V(j-1) (d tiles 2s, 2s+1) beside max / rescale decision /
  // exponentials of S(j); step 4 packs P(j); steps 4-7 S(j+1) = K(j+1).Q^T (k-step s-4).
  auto fused = [&](int j) {
    const char* vb = vring + ((j - 1) & 1) * VST;
    const char* kb = kring + ((j + 1) & 1) * KST;
    auto fetch = [&](int st, i32x4 (&F)[4]) {
      if (st < 4) {
#pragma unroll
        for (int dd = 0; dd < 2; ++dd)
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
            F[2 * dd + kc] = *reinterpret_cast<const i32x4*>(vb + voff[kc] + (2 * st + dd) * 16 * 128);
      } else {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) F[kt] = *reinterpret_cast<const i32x4*>(kb + koff[st - 4] + ktoff[kt]);
      }
    };
    i32x4 FB[2][4];
    fetch(0, FB[0]);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      i32x4 (&F)[4] = FB[st & 1];
      if (st + 1 < 8) fetch(st + 1, FB[(st + 1) & 1]);
      if (st == 0) {
        const float bm[2] = {rowmax(0), rowmax(1)};
        decide(bm);
      } else if (st == 1) {
        expo(0, 0), expo(0, 1), expo(0, 2);
      } else if (st == 2) {
        expo(0, 3), expo(1, 0), expo(1, 1);
      } else if (st == 3) {
        expo(1, 2), expo(1, 3);
      } else if (st == 4) {
        pack();
      }
      if (st < 4) {
#pragma unroll
        for (int dd = 0; dd < 2; ++dd)
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
#pragma unroll
            for (int u = 0; u < 2; ++u)
              oacc[2 * st + dd][u] = mma16<T>(as_frag(F[2 * dd + kc]), as_frag(P[u][kc]), oacc[2 * st + dd][u]);
        lsum[st >> 1] = mma16<T>(as_frag(ones), as_frag(P[st >> 1][st & 1]), lsum[st >> 1]);
      } else {
        const int ks = st - 4;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int u = 0; u < 2; ++u)
            S[kt][u] = mma16<T>(as_frag(F[kt]), qf[u][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : S[kt][u]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Block loop: the top of iteration j waits for K(j+1) and V(j-1) (issued one iteration earlier;
  // the barrier needs no full drain since nothing younger is in flight), then refills the stages
  // freed by iteration j-1.  The fused iterations form one contiguous range with a loop of its own
  // (merging both paths into one loop body costs registers).
  auto top = [&](int j) {
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8));  // vmcnt(0) lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issueK(min(j + 2, nb - 1));
    issueV(j);
  };
  auto generic = [&](int j) {
    if (j >= 1 && j - 1 < nbw) {
      rescale();
      pv(j - 1);
    }
    if (j < nbw) softmax(j, j >= nfull);
    if (j + 1 < nbw) qk(j + 1);
  };
  issueK(0);
  if (nb > 1) issueK(1);
  __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8));
  __syncthreads();
  qk(0);
  const int jf1 = max(1, min(nfull, nbw - 1));
  top(0);
  generic(0);
  int j = 1;
  for (; j < jf1; ++j) {
    top(j);
    rescale();
    fused(j);
  }
  for (; j < nb; ++j) {
    top(j);
    generic(j);
  }
  __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8));
  __syncthreads();
  if (nbw == nb) {
    rescale();
    pv(nb - 1);
  }

  // O^T accumulator: lane holds O[q0 + 16u + r16][16 dt + 4G + i]
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const float lt = lsum[u][0];
    const int qi = q0 + 16 * u + r16;
    if (qi < Lq) {
      const float inv = 1.f / lt;
      u16* orow = O + b * ql.b + h * ql.h + (int64_t)qi * ql.s;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
        i32x2 w;
        w[0] = (int)pack2<T>(oacc[dt][u][0] * inv, oacc[dt][u][1] * inv);
        w[1] = (int)pack2<T>(oacc[dt][u][2] * inv, oacc[dt][u][3] * inv);
        *reinterpret_cast<i32x2*>(orow + 16 * dt + 4 * G) = w;
      }
      if (G == 0) LSE[(int64_t)bh * Lq + qi] = (m[u] * scale2 + __log2f(lt)) * kLn2;
    }
  }
}

// ============================================================================ backward, D = 128 (MFMA 16x16x32)
// 8 bytes from LDS with the gfx950 transpose read: within each 16-lane group, lane j receives
// element j % 4 of the 8-byte pieces addressed by lanes j / 4 + 4 k, k = 0..3.  Two such reads, by
// lanes addressing rows k0 + i / 4 (+ 4) at columns m0 + 4 (i % 4), return the MFMA fragment
// A[m0 + j][k0 .. k0 + 7] of a row-major [k][m] tile: the transposed operand without a copy.
typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
Q3_DEV i32x2 ldtr(const char* p) {
  return __builtin_bit_cast(i32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)p));
}
// 16-byte chunk swizzle of the 256-byte query rows of the dK/dV tiles: a bijection onto 0..15 of
// the 16 rows a row-read pass touches ({0-3, 8-11, 16-19, 24-27}, +4), and distinct 32-byte bank
// groups for the 8 rows of each half-wave pass of a transpose read.
Q3_DEV int qswz3(int r) { return 2 * ((r & 3) | (((r >> 3) & 1) << 2)) + ((r >> 4) & 1); }

// dK/dV -- workgroup: 4 waves x 32 keys of one (b, kv head), one wave per SIMD (the K/V fragments and
// the dK/dV accumulators fill the registers); loops over the group's query heads and the 32-query
// tiles at or after the keys, Q/dO tiles and lse/delta through a 4-stage direct-to-LDS ring.  Per
// tile: S = Q K^T and dP = dO V^T (Q/dO row fragments from LDS, K/V fragments in registers),
// P = exp2(S s - lse), dS = P (dP - delta), then dV^T += dO^T P and dK^T += Q^T dS with dO^T and Q^T
// read from the same LDS tiles by transpose reads (no sequence-major copies).  MFMA row r16 of query
// tile t reads query 8 (r16/4) + 4 t + r16 % 4, so lane group G holds queries 8 G .. 8 G + 7 of each
// key: P and dS pack straight into the B operands.  Deterministic: the group's heads accumulate in
// registers.
template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_bwd_dkdv_v3(
    const u16* __restrict__ Q, Lay ql, const u16* __restrict__ K, const u16* __restrict__ V, Lay kl,
    const u16* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Delta,
    u16* __restrict__ dK, u16* __restrict__ dV, int Hq, int Hkv, int Lq, int Lk, float scale, float scale2) {
  constexpr int D = 128, BM = 32, ST = 4;
  constexpr int TB = BM * D * 2;              // one operand tile (8 KB)
  constexpr int STAGE = 2 * TB + 2 * BM * 4;  // Q, dO, lse, delta
  __shared__ __attribute__((aligned(1024))) char lds[ST * STAGE];

  const int kt = (int)blockIdx.y;  // smallest key tiles (most query tiles) first
  const int bk = blockIdx.x, b = bk / Hkv, hk = bk % Hkv, ratio = Hq / Hkv;
  const int tid = threadIdx.x, lane = tid & 63, G = lane >> 4, r16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int off = Lk - Lq;
  const int k0w = kt * 128 + wave * 32;

  // K^T / V^T B operands: lane (G, r16) holds key k0w + 16 c + r16, dims 32 ks + 8 G .. + 7
  bf16x8_t kf[2][4], vf[2][4];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int64_t row = b * kl.b + hk * kl.h + (int64_t)min(k0w + 16 * c + r16, Lk - 1) * kl.s;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kf[c][ks] = as_frag(ld16(K + row + 32 * ks + 8 * G));
      vf[c][ks] = as_frag(ld16(V + row + 32 * ks + 8 * G));
    }
  }
  f32x4 dk[8][2], dv[8][2];
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int c = 0; c < 2; ++c) dk[d][c] = dv[d][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int qstart = max(0, kt * 128 - off) / BM * BM;
  const int nq = (Lq - qstart + BM - 1) / BM;  // query tiles per head
  const int total = ratio * nq;

  auto issue = [&](int u) {  // Q and dO: 8 wave loads each (4 rows x 256 B), 2 per wave; wave 0: lse/delta
    const int hh = u / nq, q0 = qstart + (u % nq) * BM;
    const int h = hk * ratio + hh;
    const int64_t bh = (int64_t)b * Hq + h;
    const u16* Qb = Q + b * ql.b + h * ql.h;
    const u16* dOb = dO + b * ql.b + h * ql.h;
    char* base = lds + (u % ST) * STAGE;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int w = wave + 4 * i;
      const int r = 4 * w + (lane >> 4);
      const int c = (lane & 15) ^ qswz3(r);
      const int64_t src = (int64_t)min(q0 + r, Lq - 1) * ql.s + c * 8;
      __builtin_amdgcn_global_load_lds(Qb + src, (lds_vp)(base + w * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(dOb + src, (lds_vp)(base + TB + w * 1024), 16, 0, 0);
    }
    if (wave == 0) {  // lse (lanes 0..31) and delta (32..63) of the tile's queries; past Lq clamped
      const int qq = min(q0 + (lane & 31), Lq - 1);
      const float* src = (lane < 32 ? LSE : Delta) + bh * Lq + qq;
      __builtin_amdgcn_global_load_lds(src, (lds_vp)(base + 2 * TB), 4, 0, 0);
    }
  };

  // row reads: query row qrow0 (+ 4 t), chunk 4 ks + G; transpose reads: group G, lane i of read h
  // addresses query row 8 G + 4 h + i / 4, bytes 32 dt + 8 (i % 4)
  const int qrow0 = 8 * (r16 >> 2) + (r16 & 3);
  int roff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) roff[ks] = qrow0 * 256 + (((4 * ks + G) ^ qswz3(qrow0)) << 4);
  auto tr_addr = [&](int h, int dt) {
    const int row = 8 * G + 4 * h + (r16 >> 2);
    const int byte = 32 * dt + 8 * (r16 & 3);
    return row * 256 + ((((byte >> 4) ^ qswz3(row)) << 4) | (byte & 15));
  };

#pragma unroll
  for (int st = 0; st < ST - 1; ++st)
    if (st < total) issue(st);
  for (int u = 0; u < total; ++u) {
    {  // ring: tile u landed, up to ST - 2 younger tiles (4 loads per wave, 5 for wave 0) in flight
      const int younger = max(0, min(ST - 2, total - 1 - u));
      const int n = younger * (wave == 0 ? 5 : 4);
      if (n >= 10) __builtin_amdgcn_s_waitcnt((10 & 15) | (7 << 4) | (0 << 8));
      else if (n >= 8) __builtin_amdgcn_s_waitcnt((8 & 15) | (7 << 4) | (0 << 8));
      else if (n >= 5) __builtin_amdgcn_s_waitcnt((5 & 15) | (7 << 4) | (0 << 8));
      else if (n >= 4) __builtin_amdgcn_s_waitcnt((4 & 15) | (7 << 4) | (0 << 8));
      else __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8));
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (u + ST - 1 < total) issue(u + ST - 1);
    }
    const int q0 = qstart + (u % nq) * BM;
    if (min(q0 + BM - 1, Lq - 1) + off < k0w) continue;  // no query of the tile sees the wave's keys
    const char* qb = lds + (u % ST) * STAGE;
    const char* db = qb + TB;
    const float* side = reinterpret_cast<const float*>(qb + 2 * TB);
    const f32x4 l0 = *reinterpret_cast<const f32x4*>(side + 8 * G);
    const f32x4 l1 = *reinterpret_cast<const f32x4*>(side + 8 * G + 4);
    const f32x4 d0 = *reinterpret_cast<const f32x4*>(side + BM + 8 * G);
    const f32x4 d1 = *reinterpret_cast<const f32x4*>(side + BM + 8 * G + 4);

    // dP starts from -delta (its row constant), so the products leave dP - delta
    f32x4 s[2][2], dp[2][2];  // [query tile t][key tile c]
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      i32x4 qa[2], da[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        qa[t] = *reinterpret_cast<const i32x4*>(qb + roff[ks] + 4 * t * 256);
        da[t] = *reinterpret_cast<const i32x4*>(db + roff[ks] + 4 * t * 256);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          s[t][c] = mma16<T>(as_frag(qa[t]), kf[c][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[t][c]);
          dp[t][c] = mma16<T>(as_frag(da[t]), vf[c][ks], ks == 0 ? -(t ? d1 : d0) : dp[t][c]);
        }
    }
    const bool mask = !(k0w + 31 <= q0 + off && q0 + BM - 1 < Lq);
    i32x4 pp[2], dd[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float pv[8], dsv[8];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][c][i], scale2, -(t ? l1[i] : l0[i]) * kLog2e));
          if (mask) {
            const int q = q0 + 8 * G + 4 * t + i;
            p = (k0w + 16 * c + r16 <= q + off && q < Lq) ? p : 0.f;
          }
          pv[4 * t + i] = p;
          dsv[4 * t + i] = p * dp[t][c][i];
        }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        pp[c][w] = (int)pack2<T>(pv[2 * w], pv[2 * w + 1]);
        dd[c][w] = (int)pack2<T>(dsv[2 * w], dsv[2 * w + 1]);
      }
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const i32x2 q0v = ldtr(qb + tr_addr(0, dt)), q1v = ldtr(qb + tr_addr(1, dt));
      const i32x2 d0v = ldtr(db + tr_addr(0, dt)), d1v = ldtr(db + tr_addr(1, dt));
      const i32x4 aq = {q0v[0], q0v[1], q1v[0], q1v[1]}, ad = {d0v[0], d0v[1], d1v[0], d1v[1]};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        dv[dt][c] = mma16<T>(as_frag(ad), as_frag(pp[c]), dv[dt][c]);
        dk[dt][c] = mma16<T>(as_frag(aq), as_frag(dd[c]), dk[dt][c]);
      }
    }
  }

  // dK^T / dV^T accumulators: lane holds [d = 16 dt + 4 G + i][key = k0w + 16 c + r16]
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int kj = k0w + 16 * c + r16;
    if (kj >= Lk) continue;
    const int64_t row = b * kl.b + hk * kl.h + (int64_t)kj * kl.s;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      i32x2 wk, wv;
      wk[0] = (int)pack2<T>(dk[dt][c][0] * scale, dk[dt][c][1] * scale);
      wk[1] = (int)pack2<T>(dk[dt][c][2] * scale, dk[dt][c][3] * scale);
      wv[0] = (int)pack2<T>(dv[dt][c][0], dv[dt][c][1]);
      wv[1] = (int)pack2<T>(dv[dt][c][2], dv[dt][c][3]);
      *reinterpret_cast<i32x2*>(dK + row + 16 * dt + 4 * G) = wk;
      *reinterpret_cast<i32x2*>(dV + row + 16 * dt + 4 * G) = wv;
    }
  }
}

// dQ -- workgroup: 8 waves sharing one KV head, as the forward (GH query heads of the group x 8/GH
// groups of 32 query positions), 64-key blocks of K, V (rows) and K^T (the sequence-major copy)
// through a 2-stage direct-to-LDS ring.  Per block: S^T = K Q^T, dP^T = V dO^T (Q, dO fragments in
// registers), P^T = exp2(S^T s - lse), dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T; the K/V row
// mapping of the forward makes dS^T the B operand of the K^T product as it comes out.
template <typename T, int GH>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_bwd_dq_v3(
    const u16* __restrict__ Q, Lay ql, const u16* __restrict__ K, const u16* __restrict__ V, Lay kl,
    const u16* __restrict__ Kt, const u16* __restrict__ dO, const float* __restrict__ LSE,
    const float* __restrict__ Delta, u16* __restrict__ dQ, int Hq, int Hkv, int Lq, int Lk, int ldkt, float scale,
    float scale2) {
  constexpr int D = 128, BN = 64, NW = 8, QT = 32 * (NW / GH);
  constexpr int KST = BN * D * 2;  // one 64 x 128 tile
  constexpr int STAGE = 3 * KST;   // K, V, K^T
  __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE];

  const int nqt = (Lq + QT - 1) / QT;
  const int qt = nqt - 1 - (int)blockIdx.y;  // longest query tiles first
  const int tid = threadIdx.x, lane = tid & 63, G = lane >> 4, r16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int HB = Hq / GH, b = (int)blockIdx.x / HB, h = ((int)blockIdx.x % HB) * GH + wave % GH;
  const int hk = h / (Hq / Hkv), bh = b * Hq + h;
  const int off = Lk - Lq;
  const int q0 = qt * QT + (wave / GH) * 32;
  const u16* Kb = K + b * kl.b + hk * kl.h;
  const u16* Vb = V + b * kl.b + hk * kl.h;
  const u16* Ktb = Kt + (int64_t)(b * Hkv + hk) * D * ldkt;

  bf16x8_t qf[2][4], df[2][4];
  float lse2[2], dlt[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int qi = min(q0 + 16 * u + r16, Lq - 1);
    const int64_t row = b * ql.b + h * ql.h + (int64_t)qi * ql.s;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[u][ks] = as_frag(ld16(Q + row + 32 * ks + 8 * G));
      df[u][ks] = as_frag(ld16(dO + row + 32 * ks + 8 * G));
    }
    lse2[u] = LSE[(int64_t)bh * Lq + qi] * kLog2e;
    dlt[u] = Delta[(int64_t)bh * Lq + qi];
  }

  const int nb = (min(Lk, min(qt * QT + QT - 1, Lq - 1) + off + 1) + BN - 1) / BN;
  const int nbw = min(nb, (min(Lk, min(q0 + 31, Lq - 1) + off + 1) + BN - 1) / BN);
  const int nfull = min(nbw, max(0, (q0 + off + 1) / BN));  // blocks fully visible to the wave
  const int qpos[2] = {q0 + r16 + off, q0 + 16 + r16 + off};

  auto issue = [&](int j) {  // K, V: 16 wave loads each (4 rows x 256 B); K^T: 16 (8 rows x 128 B)
    const int k0 = j * BN;
    char* base = lds + (j & 1) * STAGE;
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i) {
      const int w = wave + NW * i;
      const int r = w * 4 + (lane >> 4);
      const int c = (lane & 15) ^ kswz3(r);
      const int64_t src = (int64_t)min(k0 + r, Lk - 1) * kl.s + c * 8;
      __builtin_amdgcn_global_load_lds(Kb + src, (lds_vp)(base + w * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(Vb + src, (lds_vp)(base + KST + w * 1024), 16, 0, 0);
      const int rt = w * 8 + (lane >> 3);
      const int ct = (lane & 7) ^ vswz3(rt);
      __builtin_amdgcn_global_load_lds(Ktb + (int64_t)rt * ldkt + min(k0 + ct * 8, ldkt - 8),
                                       (lds_vp)(base + 2 * KST + w * 1024), 16, 0, 0);
    }
  };

  const int krow0 = 4 * ((r16 >> 2) & 1) + 16 * (r16 >> 3) + (r16 & 3);
  const int kbase = 4 * (G & 1) + 16 * (G >> 1);
  int koff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) koff[ks] = krow0 * 256 + (((4 * ks + G) ^ r16) << 4);
  int toff[2];
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) toff[kc] = r16 * 128 + (((4 * kc + G) ^ vswz3(r16)) << 4);
  constexpr int ktoff[4] = {0, 8 * 256, 32 * 256, 40 * 256};

  f32x4 dq[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int u = 0; u < 2; ++u) dq[dt][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  issue(0);
  for (int j = 0; j < nb; ++j) {
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0 << 8));  // block j landed; nothing younger
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (j + 1 < nb) issue(j + 1);
    if (j >= nbw) continue;
    const char* kb = lds + (j & 1) * STAGE;
    const char* vb = kb + KST;
    const char* tb = kb + 2 * KST;
    f32x4 S[4][2], DP[4][2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(kb + koff[ks] + ktoff[kt]);
        const i32x4 av = *reinterpret_cast<const i32x4*>(vb + koff[ks] + ktoff[kt]);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          S[kt][u] = mma16<T>(as_frag(a), qf[u][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : S[kt][u]);
          DP[kt][u] = mma16<T>(as_frag(av), df[u][ks], ks == 0 ? f32x4{-dlt[u], -dlt[u], -dlt[u], -dlt[u]} : DP[kt][u]);
        }
      }
    const bool mask = j >= nfull;
    i32x4 DS[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int qrel = qpos[u] - j * BN - kbase;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(S[kt][u][i], scale2, -lse2[u]));
          if (mask) p = 32 * (kt >> 1) + 8 * (kt & 1) + i <= qrel ? p : 0.f;
          S[kt][u][i] = p * DP[kt][u][i];  // DP started from -delta
        }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        i32x4 w;
        w[0] = (int)pack2<T>(S[2 * c][u][0], S[2 * c][u][1]);
        w[1] = (int)pack2<T>(S[2 * c][u][2], S[2 * c][u][3]);
        w[2] = (int)pack2<T>(S[2 * c + 1][u][0], S[2 * c + 1][u][1]);
        w[3] = (int)pack2<T>(S[2 * c + 1][u][2], S[2 * c + 1][u][3]);
        DS[u][c] = w;
      }
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const i32x4 a = *reinterpret_cast<const i32x4*>(tb + toff[kc] + dt * 16 * 128);
#pragma unroll
        for (int u = 0; u < 2; ++u) dq[dt][u] = mma16<T>(as_frag(a), as_frag(DS[u][kc]), dq[dt][u]);
      }
  }

  // dQ^T accumulator: lane holds dQ[q0 + 16 u + r16][16 dt + 4 G + i]
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int qi = q0 + 16 * u + r16;
    if (qi >= Lq) continue;
    u16* row = dQ + b * ql.b + h * ql.h + (int64_t)qi * ql.s;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      i32x2 w;
      w[0] = (int)pack2<T>(dq[dt][u][0] * scale, dq[dt][u][1] * scale);
      w[1] = (int)pack2<T>(dq[dt][u][2] * scale, dq[dt][u][3] * scale);
      *reinterpret_cast<i32x2*>(row + 16 * dt + 4 * G) = w;
    }
  }
}

// ============================================================================ backward: delta
// delta[r] = sum_d O[r,d] * dO[r,d] (fp32), one wave per row.
template <typename T>
__global__ __launch_bounds__(kThreads) void attn_delta_kernel(const typename T::storage* __restrict__ O,
                                                              const typename T::storage* __restrict__ dO, Lay ql,
                                                              float* __restrict__ delta, int64_t rows, int H, int L,
                                                              int D) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t b = row / ((int64_t)H * L), h = (row / L) % H, q = row % L;
  const int64_t base = b * ql.b + h * ql.h + q * ql.s;
  float s = 0.f;
  for (int d = lane_id(); d < D; d += 64) s += to_f32<T>(O[base + d]) * to_f32<T>(dO[base + d]);
  s = group_sum<64>(s);
  if (lane_id() == 0) delta[row] = s;
}

// Vectorised delta: LPR = D / 8 lanes per row, 16 bytes of O and dO per lane (one row per LPR-lane
// group, 64 / LPR rows per wave); the row sum is a DPP reduction over the group.
template <typename T, int LPR>
__global__ __launch_bounds__(kThreads) void attn_delta_vec_kernel(const typename T::storage* __restrict__ O,
                                                                  const typename T::storage* __restrict__ dO,
                                                                  Lay ql, float* __restrict__ delta, int64_t rows,
                                                                  int H, int L) {
  constexpr int RPW = 64 / LPR;
  const int lane = lane_id(), sub = lane % LPR;
  const int64_t row = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * RPW + lane / LPR;
  const int64_t rc = row < rows ? row : rows - 1;
  const int64_t b = rc / ((int64_t)H * L), h = (rc / L) % H, q = rc % L;
  const int64_t base = b * ql.b + h * ql.h + q * ql.s + sub * 8;
  const Vec<T> o = load_vec<T>(O + base), g = load_vec<T>(dO + base);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += o.v[e] * g.v[e];
  s = group_sum<LPR>(s);
  if (sub == 0 && row < rows) delta[row] = s;
}

// ============================================================================ backward (MFMA)
// dQ kernel -- workgroup: 4 waves x 32 queries of one (b, h).  Per 64-key tile: S^T = K Q^T,
// dP^T = V dO^T, dS = P (dP - delta), dQ^T += Kt dS^T.
// dK/dV kernel -- workgroup: 4 waves x 32 keys of one (b, kv head); loops over the Hq/Hkv query
// heads of the group and the 32-query tiles at or after the diagonal.  Per tile: S = Q K^T,
// dP = dO V^T (lane = key), P, dS; dV^T += dOt P, dK^T += Qt dS.  The group's query heads
// accumulate into the same registers: no partial buffers, no atomics, deterministic.
// Operand tiles move global -> LDS with wave-wide global_load_lds_dwordx4 into swizzled, unpadded
// LDS rows (no register staging); two waves per SIMD except dK/dV at D = 128 (its K/V fragments and
// two accumulators need the full register file); causal masks only on tiles that cross the diagonal, and
// the grid is ordered longest-work-first.
template <typename T, int D, int STAGES>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_bwd_dq_v2(
    const u16* __restrict__ Q, Lay ql, const u16* __restrict__ K, const u16* __restrict__ V, Lay kl,
    const u16* __restrict__ Kt, const u16* __restrict__ dO, const float* __restrict__ LSE,
    const float* __restrict__ Delta, u16* __restrict__ dQ, int Hq, int Hkv, int Lq, int Lk, int ldkt, float scale,
    float scale2) {
  constexpr int BN = 64, KS = D / 16, DT = D / 32;
  constexpr int CPK = D / 8, RPK = 64 / CPK, CPV = BN / 8, RPV = 64 / CPV;
  constexpr int KLOADS = BN / RPK, TLOADS = D / RPV;
  constexpr int NLOADS = 2 * KLOADS + TLOADS;
  static_assert(NLOADS % 4 == 0, "loads split over 4 waves");
  constexpr int LPW = NLOADS / 4;
  constexpr int KB = BN * D * 2, STAGE = 2 * KB + D * BN * 2;
  __shared__ __attribute__((aligned(1024))) char lds[STAGES * STAGE];

  const int nqt = (Lq + 127) / 128;
  const int qt = nqt - 1 - (int)blockIdx.y;  // longest query tiles first
  const int bh = blockIdx.x, b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hkv);
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int off = Lk - Lq;
  const int q0 = qt * 128 + wave * 32;
  const int qi = q0 + (lane & 31);
  const u16* Kb = K + b * kl.b + hk * kl.h;
  const u16* Vb = V + b * kl.b + hk * kl.h;
  const u16* Ktb = Kt + (int64_t)(b * Hkv + hk) * D * ldkt;
  const int64_t qrow = b * ql.b + h * ql.h + (int64_t)min(qi, Lq - 1) * ql.s;

  bf16x8_t qf[KS], dof[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = as_frag(ld16(Q + qrow + ks * 16 + g * 8));
    dof[ks] = as_frag(ld16(dO + qrow + ks * 16 + g * 8));
  }
  const float lse2 = qi < Lq ? LSE[(int64_t)bh * Lq + qi] * kLog2e : 0.f;
  const float dlt = qi < Lq ? Delta[(int64_t)bh * Lq + qi] : 0.f;
  const int qpos = qi + off;
  const int qlast_blk = min(qt * 128 + 127, Lq - 1) + off;
  const int ntiles = (min(Lk, qlast_blk + 1) + BN - 1) / BN;
  const int qfirst_wave = q0 + off;
  const int qlast_wave = min(q0 + 31, Lq - 1) + off;

  auto issue = [&](int stage, int t) {
    const int k0 = t * BN;
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int w = wave + 4 * i;
      const void* src;
      int dst;
      if (w < 2 * KLOADS) {
        const int which = w / KLOADS, wl = w % KLOADS;
        const int r = wl * RPK + lane / CPK;
        const int c = (lane % CPK) ^ chunk_swz<CPK>(r);
        src = (which ? Vb : Kb) + (int64_t)min(k0 + r, Lk - 1) * kl.s + c * 8;
        dst = stage * STAGE + which * KB + wl * RPK * D * 2;
      } else {
        const int wl = w - 2 * KLOADS;
        const int r = wl * RPV + lane / CPV;
        const int c = (lane % CPV) ^ chunk_swz<CPV>(r);
        src = Ktb + (int64_t)r * ldkt + min(k0 + c * 8, ldkt - 8);
        dst = stage * STAGE + 2 * KB + wl * RPV * BN * 2;
      }
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(lds + dst), 16, 0, 0);
    }
  };

  f32x16 dq[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) dq[i] = zero16();
  const int kr = lane & 31;
  const int ksw = chunk_swz<CPK>(kr), ksw2 = chunk_swz<CPK>(kr + 32);

#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st)
    if (st < ntiles) issue(st, st);
  for (int t = 0; t < ntiles; ++t) {
    if constexpr (STAGES == 1) {
      __syncthreads();  // everyone is done reading the single stage
      issue(0, t);
    }
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));  // vmcnt(0)
    __syncthreads();
    if constexpr (STAGES > 1) {
      if (t + STAGES - 1 < ntiles) issue((t + STAGES - 1) % STAGES, t + STAGES - 1);
    }
    const int k0 = t * BN;
    if (k0 > qlast_wave) continue;
    const char* kb = lds + (t % STAGES) * STAGE;
    const char* vb = kb + KB;
    const char* tb = kb + 2 * KB;
    const bool full = k0 + BN - 1 <= qfirst_wave && q0 + 31 < Lq;
#pragma nounroll
    for (int tt = 0; tt < 2; ++tt) {  // two 32-key halves keep only one score tile live
      f32x16 sc = zero16(), dp = zero16();
      const int kro = kr + tt * 32, kswt = tt ? ksw2 : ksw;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int o = kro * D * 2 + (((ks * 2 + g) ^ kswt) << 4);
        sc = mma<T>(as_frag(*reinterpret_cast<const i32x4*>(kb + o)), qf[ks], sc);
        dp = mma<T>(as_frag(*reinterpret_cast<const i32x4*>(vb + o)), dof[ks], dp);
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = k0 + tt * 32 + acc_row(v, lane);
        float p = __builtin_amdgcn_exp2f(sc[v] * scale2 - lse2);
        if (!full) p = key <= qpos ? p : 0.f;
        sc[v] = p * (dp[v] - dlt);
      }
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const int c = tt * 2 + c2;
        const bf16x8_t db = pack8<T>(sc, c2 * 8);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int r = dt * 32 + (lane & 31);
          const char* row = tb + r * BN * 2;
          const i32x4 v4 = *reinterpret_cast<const i32x4*>(row + (((2 * c + g) ^ chunk_swz<CPV>(r)) << 4));
          dq[dt] = mma<T>(as_frag(v4), db, dq[dt]);
        }
      }
    }
  }
  if (qi < Lq) {
    u16* row = dQ + qrow;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int d = dt * 32 + 8 * vg + 4 * g;
        typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
        i32x2 w;
        w[0] = (int)pack2<T>(dq[dt][4 * vg] * scale, dq[dt][4 * vg + 1] * scale);
        w[1] = (int)pack2<T>(dq[dt][4 * vg + 2] * scale, dq[dt][4 * vg + 3] * scale);
        *reinterpret_cast<i32x2*>(row + d) = w;
      }
  }
}

template <typename T, int D, int OCC, int STAGES>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void attn_bwd_dkdv_v2(
    const u16* __restrict__ Q, Lay ql, const u16* __restrict__ K, const u16* __restrict__ V, Lay kl,
    const u16* __restrict__ Qt, const u16* __restrict__ dO, const u16* __restrict__ dOt,
    const float* __restrict__ LSE, const float* __restrict__ Delta, u16* __restrict__ dK, u16* __restrict__ dV,
    int Hq, int Hkv, int Lq, int Lk, int ldqt, float scale, float scale2) {
  constexpr int BM = 32, KS = D / 16, DT = D / 32;
  constexpr int CPK = D / 8, RPK = 64 / CPK, CPQ = BM / 8, RPQ = 64 / CPQ;
  constexpr int QLOADS = BM / RPK, TLOADS = D / RPQ;
  constexpr int NLOADS = 2 * QLOADS + 2 * TLOADS;
  static_assert(NLOADS % 4 == 0, "loads split over 4 waves");
  constexpr int LPW = NLOADS / 4;
  constexpr int QB = BM * D * 2, STAGE = 4 * QB + 2 * BM * 4;
  // D = 128: the V fragments of each wave's 32 keys live in a wave-private LDS block instead of
  // registers (the two 128-register accumulators and the K fragments fill the VGPRs; with V also
  // resident the compiler parked it in AGPRs and copied it back, and had no registers left to
  // prefetch LDS operands).  Each lane reads back exactly the 16-byte chunks it wrote.
  constexpr bool VLDS = D == 128;
  constexpr int VBYTES = VLDS ? 4 * 32 * D * 2 : 16;
  __shared__ __attribute__((aligned(1024))) char lds[STAGES * STAGE + VBYTES];

  const int kt = (int)blockIdx.y;  // smallest key tiles (the most query tiles) first
  const int bk = blockIdx.x, b = bk / Hkv, hk = bk % Hkv, ratio = Hq / Hkv;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int off = Lk - Lq;
  const int k0w = kt * 128 + wave * 32;
  const int kj = k0w + (lane & 31);
  const int64_t krow = b * kl.b + hk * kl.h + (int64_t)min(kj, Lk - 1) * kl.s;

  bf16x8_t kf[KS], vf[VLDS ? 1 : KS];
  char* vblk = lds + STAGES * STAGE + wave * 32 * D * 2 + (lane & 31) * D * 2;  // this lane's key row
  auto voff = [&](int ks) { return ((2 * ks + g) ^ chunk_swz<CPK>(lane & 31)) << 4; };
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kf[ks] = as_frag(ld16(K + krow + ks * 16 + g * 8));
    if constexpr (VLDS) *reinterpret_cast<i32x4*>(vblk + voff(ks)) = ld16(V + krow + ks * 16 + g * 8);
    else vf[ks] = as_frag(ld16(V + krow + ks * 16 + g * 8));
  }
  auto vfrag = [&](int ks) {
    if constexpr (VLDS) return as_frag(*(const volatile __attribute__((address_space(3))) i32x4*)(vblk + voff(ks)));
    else return vf[ks];
  };
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) dk[i] = dv[i] = zero16();

  const int qstart = max(0, kt * 128 - off) / BM * BM;
  const int nq = (Lq - qstart + BM - 1) / BM;  // query tiles per head
  const int total = ratio * nq;

  // D = 128, full query tile (q0 + BM <= Lq): load i (0, 1) of each operand covers rows
  // wl * RPK + lane / CPK (wl = wave + 4 i) of Q and dO, rows wl * RPQ + lane / CPQ of Q^T and dO^T;
  // per-lane byte offsets precomputed here, wave-uniform tile bases added per tile.
  auto qoff = [&](int i) {
    const int r = (wave + 4 * i) * RPK + lane / CPK;
    return (uint32_t)(((int64_t)r * ql.s + ((lane % CPK) ^ chunk_swz<CPK>(r)) * 8) * 2);
  };
  auto toff = [&](int i) {
    const int r = (wave + 4 * i) * RPQ + lane / CPQ;
    return (uint32_t)(((int64_t)r * ldqt + ((lane % CPQ) ^ chunk_swz<CPQ>(r)) * 8) * 2);
  };
  // 32-bit lane offsets: bounded strides keep them exact
  const bool kFast = D == 128 && ldqt < (1 << 24) && ql.s < (1 << 24);
  static_assert(D != 128 || (QLOADS == 8 && TLOADS == 8 && LPW == 8), "load schedule of the D = 128 tile");
  const uint32_t qo0 = qoff(0), qo1 = qoff(1), to0 = toff(0), to1 = toff(1);

  // tile u = (head hh, query tile): operands Q, dO rows and Q^T, dO^T columns, plus lse/delta
  auto issue = [&](int stage, int u) {
    const int hh = u / nq, q0 = qstart + (u % nq) * BM;
    const int h = hk * ratio + hh;
    const int64_t bh = (int64_t)b * Hq + h;
    const u16* Qb = Q + b * ql.b + h * ql.h;
    const u16* dOb = dO + b * ql.b + h * ql.h;
    const u16* Qtb = Qt + bh * D * ldqt;
    const u16* dOtb = dOt + bh * D * ldqt;
    if (kFast && q0 + BM <= Lq) {
      const char* qs = reinterpret_cast<const char*>(Qb + (int64_t)q0 * ql.s);
      const char* ds = reinterpret_cast<const char*>(dOb + (int64_t)q0 * ql.s);
      const char* qts = reinterpret_cast<const char*>(Qtb + q0);
      const char* dts = reinterpret_cast<const char*>(dOtb + q0);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int wl = wave + 4 * i;
        const uint32_t qo = i ? qo1 : qo0, to = i ? to1 : to0;
        __builtin_amdgcn_global_load_lds(qs + qo, (lds_vp)(lds + stage * STAGE + wl * RPK * D * 2), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(ds + qo, (lds_vp)(lds + stage * STAGE + QB + wl * RPK * D * 2), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(qts + to, (lds_vp)(lds + stage * STAGE + 2 * QB + wl * RPQ * BM * 2), 16,
                                         0, 0);
        __builtin_amdgcn_global_load_lds(dts + to, (lds_vp)(lds + stage * STAGE + 3 * QB + wl * RPQ * BM * 2), 16,
                                         0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int w = wave + 4 * i;
        const void* src;
        int dst;
        if (w < 2 * QLOADS) {
          const int which = w / QLOADS, wl = w % QLOADS;
          const int r = wl * RPK + lane / CPK;
          const int c = (lane % CPK) ^ chunk_swz<CPK>(r);
          src = (which ? dOb : Qb) + (int64_t)min(q0 + r, Lq - 1) * ql.s + c * 8;
          dst = stage * STAGE + which * QB + wl * RPK * D * 2;
        } else {
          const int which = (w - 2 * QLOADS) / TLOADS, wl = (w - 2 * QLOADS) % TLOADS;
          const int r = wl * RPQ + lane / CPQ;
          const int c = (lane % CPQ) ^ chunk_swz<CPQ>(r);
          src = (which ? dOtb : Qtb) + (int64_t)r * ldqt + min(q0 + c * 8, ldqt - 8);
          dst = stage * STAGE + (2 + which) * QB + wl * RPQ * BM * 2;
        }
        __builtin_amdgcn_global_load_lds(src, (lds_vp)(lds + dst), 16, 0, 0);
      }
    }
    // lse (lanes 0..31) and delta (lanes 32..63) of the tile's queries, straight into LDS like the
    // operand tiles (a plain load + LDS store would stall wave 0 for a memory round trip per tile);
    // queries past Lq read a clamped row and are masked where used.
    static_assert(BM == 32, "side vector layout");
    if (wave == 0) {
      const int qq = min(q0 + (lane & 31), Lq - 1);
      const float* src = (lane < 32 ? LSE : Delta) + bh * Lq + qq;
      __builtin_amdgcn_global_load_lds(src, (lds_vp)(lds + stage * STAGE + 4 * QB), 4, 0, 0);
    }
  };

  // STAGES-deep ring: tiles u+1 .. u+STAGES-1 are in flight while tile u is computed.  Wave 0 issues
  // one more load per tile (the lse/delta vector) than the others.
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st)
    if (st < total) issue(st, st);
  for (int u = 0; u < total; ++u) {
    const int younger = min(STAGES - 2, total - 1 - u);
    if (wave == 0) ring_wait<LPW + 1>(younger);
    else ring_wait<LPW>(younger);
    if (u + STAGES - 1 < total) issue((u + STAGES - 1) % STAGES, u + STAGES - 1);
    const int q0 = qstart + (u % nq) * BM;
    if (min(q0 + BM - 1, Lq - 1) + off < k0w) continue;  // no query of the tile sees the wave's keys
    const char* qb = lds + (u % STAGES) * STAGE;
    const char* db = qb + QB;
    const char* qtb = qb + 2 * QB;
    const char* dtb = qb + 3 * QB;
    const float* side = reinterpret_cast<const float*>(qb + 4 * QB);
    f32x16 s = zero16(), dp = zero16();
    const int qr = lane & 31, qsw = chunk_swz<CPK>(qr);
    // Operand fragments one k-step ahead: step ks+1's LDS reads are issued before step ks's MFMAs
    // (scheduling fences keep the order), so a read's latency overlaps the previous MFMAs.
    auto qoffs = [&](int ks) { return qr * D * 2 + (((ks * 2 + g) ^ qsw) << 4); };
    // volatile: the reads keep program order (prologue before prefetch), so each wait covers
    // exactly the fragments the next MFMAs use
    auto rd = [](const char* p) { return *(const volatile __attribute__((address_space(3))) i32x4*)(p); };
    i32x4 fq[2], fd[2];
    bf16x8_t fv[2];
    fq[0] = rd(qb + qoffs(0));
    fd[0] = rd(db + qoffs(0));
    fv[0] = vfrag(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) {
        fq[cur ^ 1] = rd(qb + qoffs(ks + 1));
        fd[cur ^ 1] = rd(db + qoffs(ks + 1));
        fv[cur ^ 1] = vfrag(ks + 1);
      }
      if (ks + 1 < KS) __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (3 << 8) | (3 << 14));  // lgkmcnt(3)
      __builtin_amdgcn_sched_barrier(0);
      s = mma<T>(as_frag(fq[cur]), kf[ks], s);
      dp = mma<T>(as_frag(fd[cur]), fv[cur], dp);
      __builtin_amdgcn_sched_barrier(0);
    }
    const bool full = k0w + 31 <= q0 + off && q0 + BM - 1 < Lq;
    f32x16 ds;
    if (full) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = acc_row(v, lane);
        const float p = __builtin_amdgcn_exp2f(s[v] * scale2 - side[r] * kLog2e);
        s[v] = p;
        ds[v] = p * (dp[v] - side[BM + r]);
      }
    } else {
      // query q0 + r is kept when r in [lo, hi): at or after the lane's key (causal) and inside Lq
      const int lo = kj - off - q0, hi = Lq - q0;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = acc_row(v, lane);
        float p = __builtin_amdgcn_exp2f(s[v] * scale2 - side[r] * kLog2e);
        p = (r >= lo && r < hi) ? p : 0.f;
        s[v] = p;
        ds[v] = p * (dp[v] - side[BM + r]);
      }
    }
    // dV^T += dO^T P and dK^T += Q^T dS over the tile's 32 queries: (c, dt) pairs in order, the next
    // pair's two fragments read before the current pair's MFMAs.
    const bf16x8_t pk[2] = {pack8<T>(s, 0), pack8<T>(s, 8)};
    const bf16x8_t dk8[2] = {pack8<T>(ds, 0), pack8<T>(ds, 8)};
    auto toffs = [&](int c, int dt) {
      const int r = dt * 32 + (lane & 31);
      return r * BM * 2 + (((2 * c + g) ^ chunk_swz<CPQ>(r)) << 4);
    };
    constexpr int NP = (BM / 16) * DT;
    i32x4 fa[2], fb[2];
    fa[0] = rd(dtb + toffs(0, 0));
    fb[0] = rd(qtb + toffs(0, 0));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int pi = 0; pi < NP; ++pi) {
      const int c = pi / DT, dt = pi % DT, cur = pi & 1;
      if (pi + 1 < NP) {
        const int o = toffs((pi + 1) / DT, (pi + 1) % DT);
        fa[cur ^ 1] = rd(dtb + o);
        fb[cur ^ 1] = rd(qtb + o);
      }
      // the pair's fragments landed; the next pair's two reads may still be in flight
      if (pi + 1 < NP) __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (2 << 8) | (3 << 14));  // lgkmcnt(2)
      __builtin_amdgcn_sched_barrier(0);
      dv[dt] = mma<T>(as_frag(fa[cur]), pk[c], dv[dt]);
      dk[dt] = mma<T>(as_frag(fb[cur]), dk8[c], dk[dt]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (kj < Lk) {
    u16* kout = dK + krow;
    u16* vout = dV + krow;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int d = dt * 32 + 8 * vg + 4 * g;
        typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
        i32x2 wk, wv;
        wk[0] = (int)pack2<T>(dk[dt][4 * vg] * scale, dk[dt][4 * vg + 1] * scale);
        wk[1] = (int)pack2<T>(dk[dt][4 * vg + 2] * scale, dk[dt][4 * vg + 3] * scale);
        wv[0] = (int)pack2<T>(dv[dt][4 * vg], dv[dt][4 * vg + 1]);
        wv[1] = (int)pack2<T>(dv[dt][4 * vg + 2], dv[dt][4 * vg + 3]);
        *reinterpret_cast<i32x2*>(kout + d) = wk;
        *reinterpret_cast<i32x2*>(vout + d) = wv;
      }
  }
}

// ============================================================================ SIMT path
// One wave per (b, h, query) or (b, kv head, key); D <= 256 with lane holding d = lane + 64*i.
template <typename T>
__global__ __launch_bounds__(kThreads) void attn_fwd_simt(const typename T::storage* __restrict__ Q, Lay ql,
                                                          const typename T::storage* __restrict__ K,
                                                          const typename T::storage* __restrict__ V, Lay kl,
                                                          typename T::storage* __restrict__ O,
                                                          float* __restrict__ LSE, int Hq, int Hkv, int Lq, int Lk,
                                                          int D, float scale) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.z;
  if (row >= (int64_t)Hq * Lq) return;
  const int h = (int)(row / Lq), qi = (int)(row % Lq), hk = h / (Hq / Hkv), l = lane_id();
  const int64_t bh = (int64_t)b * Hq + h;
  const int64_t qrow = b * ql.b + h * ql.h + qi * ql.s;
  const typename T::storage* kb = K + b * kl.b + hk * kl.h;
  const typename T::storage* vb = V + b * kl.b + hk * kl.h;
  float qv[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) qv[i] = (l + 64 * i < D) ? to_f32<T>(Q[qrow + l + 64 * i]) : 0.f;
  float m = -INFINITY, den = 0.f;
  const int kend = min(Lk, qi + (Lk - Lq) + 1);
  for (int j = 0; j < kend; ++j) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (l + 64 * i < D) s += qv[i] * to_f32<T>(kb[j * kl.s + l + 64 * i]);
    s = group_sum<64>(s) * scale;
    const float mn = fmaxf(m, s), a = __expf(m - mn), p = __expf(s - mn);
    den = den * a + p;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (l + 64 * i < D) acc[i] = acc[i] * a + p * to_f32<T>(vb[j * kl.s + l + 64 * i]);
    m = mn;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (l + 64 * i < D) O[qrow + l + 64 * i] = from_f32<T>(acc[i] / den);
  if (l == 0) LSE[bh * Lq + qi] = m + __logf(den);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void attn_bwd_dq_simt(const typename T::storage* __restrict__ Q, Lay ql,
                                                             const typename T::storage* __restrict__ K,
                                                             const typename T::storage* __restrict__ V, Lay kl,
                                                             const typename T::storage* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             const float* __restrict__ Delta,
                                                             typename T::storage* __restrict__ dQ, int Hq, int Hkv,
                                                             int Lq, int Lk, int D, float scale) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.z;
  if (row >= (int64_t)Hq * Lq) return;
  const int h = (int)(row / Lq), qi = (int)(row % Lq), hk = h / (Hq / Hkv), l = lane_id();
  const int64_t bh = (int64_t)b * Hq + h;
  const int64_t qrow = b * ql.b + h * ql.h + qi * ql.s;
  const typename T::storage* kb = K + b * kl.b + hk * kl.h;
  const typename T::storage* vb = V + b * kl.b + hk * kl.h;
  float qv[4], dov[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = l + 64 * i < D;
    qv[i] = ok ? to_f32<T>(Q[qrow + l + 64 * i]) : 0.f;
    dov[i] = ok ? to_f32<T>(dO[qrow + l + 64 * i]) : 0.f;
  }
  const float lse = LSE[bh * Lq + qi], dl = Delta[bh * Lq + qi];
  const int kend = min(Lk, qi + (Lk - Lq) + 1);
  for (int j = 0; j < kend; ++j) {
    float s = 0.f, dp = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (l + 64 * i < D) {
        s += qv[i] * to_f32<T>(kb[j * kl.s + l + 64 * i]);
        dp += dov[i] * to_f32<T>(vb[j * kl.s + l + 64 * i]);
      }
    s = group_sum<64>(s);
    dp = group_sum<64>(dp);
    const float p = __expf(s * scale - lse), ds = p * (dp - dl);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (l + 64 * i < D) acc[i] += ds * to_f32<T>(kb[j * kl.s + l + 64 * i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (l + 64 * i < D) dQ[qrow + l + 64 * i] = from_f32<T>(acc[i] * scale);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void attn_bwd_dkdv_simt(const typename T::storage* __restrict__ Q, Lay ql,
                                                               const typename T::storage* __restrict__ K,
                                                               const typename T::storage* __restrict__ V, Lay kl,
                                                               const typename T::storage* __restrict__ dO,
                                                               const float* __restrict__ LSE,
                                                               const float* __restrict__ Delta,
                                                               typename T::storage* __restrict__ dK,
                                                               typename T::storage* __restrict__ dV, int Hq, int Hkv,
                                                               int Lq, int Lk, int D, float scale) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.z;
  if (row >= (int64_t)Hkv * Lk) return;
  const int hk = (int)(row / Lk), kj = (int)(row % Lk), ratio = Hq / Hkv, l = lane_id();
  const int64_t krow = b * kl.b + hk * kl.h + kj * kl.s;
  float kv[4], vv[4], ak[4] = {0.f, 0.f, 0.f, 0.f}, av[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = l + 64 * i < D;
    kv[i] = ok ? to_f32<T>(K[krow + l + 64 * i]) : 0.f;
    vv[i] = ok ? to_f32<T>(V[krow + l + 64 * i]) : 0.f;
  }
  const int off = Lk - Lq;
  for (int hh = 0; hh < ratio; ++hh) {
    const int h = hk * ratio + hh;
    const int64_t bh = (int64_t)b * Hq + h;
    for (int qi = max(0, kj - off); qi < Lq; ++qi) {
      const typename T::storage* q = Q + b * ql.b + h * ql.h + qi * ql.s;
      const typename T::storage* d = dO + b * ql.b + h * ql.h + qi * ql.s;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (l + 64 * i < D) {
          s += kv[i] * to_f32<T>(q[l + 64 * i]);
          dp += vv[i] * to_f32<T>(d[l + 64 * i]);
        }
      s = group_sum<64>(s);
      dp = group_sum<64>(dp);
      const float p = __expf(s * scale - LSE[bh * Lq + qi]), ds = p * (dp - Delta[bh * Lq + qi]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (l + 64 * i < D) {
          av[i] += p * to_f32<T>(d[l + 64 * i]);
          ak[i] += ds * to_f32<T>(q[l + 64 * i]);
        }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (l + 64 * i < D) {
      dK[krow + l + 64 * i] = from_f32<T>(ak[i] * scale);
      dV[krow + l + 64 * i] = from_f32<T>(av[i]);
    }
}

// ============================================================================ sequence-major copy
// y[(b*H + h)*D + d][p] = x[b*sb + h*sh + perm16(p)*ss + d] (0 where perm16(p) >= L): the
// sequence-contiguous operand copies of the matrix-core path, with the 4-position groups 1 and 2
// of every 16-position block swapped.  A lane's operand slice of such a row -- positions
// {16c + 4g .. +3} and {16c + 8 + 4g .. +3}, the order in which the 32x32 accumulator layout hands
// over P and dS -- is then one contiguous 16-byte chunk (8 + 8 bytes would read at half rate).
// 64 x 64 (position x d) LDS tiles.
Q3_DEV int perm16(int p) { return p ^ ((((p >> 2) ^ (p >> 3)) & 1) * 12); }
__global__ __launch_bounds__(kThreads) void seq_major_kernel(const u16* __restrict__ x, Lay xl, u16* __restrict__ y,
                                                             int64_t ldy, int H, int L, int D) {
  __shared__ u16 tile[64][66];
  const int bh = blockIdx.z, b = bh / H, h = bh % H;
  const int s0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const u16* xb = x + b * xl.b + h * xl.h;
  for (int r = ty; r < 64; r += 4) {
    const int s = s0 + r, d = d0 + tx;
    tile[r][tx] = (s < L && d < D) ? xb[s * xl.s + d] : (u16)0;
  }
  __syncthreads();
  u16* yb = y + (int64_t)bh * D * ldy;
  for (int c = ty; c < 64; c += 4) {
    const int d = d0 + c, s = s0 + tx;
    if (d < D && s < ldy) yb[(int64_t)d * ldy + s] = tile[perm16(tx)][c];
  }
}

// Vectorised form (D % 64 == 0, 16-byte aligned rows): a wave covers 64 output positions x 64 d;
// lane (dc = lane % 8, sg = lane / 8) loads the 8 source rows of output positions p0 .. p0 + 7
// (p0 = 8 sg, rows perm16(p)) at d0 + 8 dc .. + 7 (16 bytes each), transposes the 8 x 8 block in
// registers and writes 8 d rows x 16 bytes.  Loads are 128-byte row segments, stores 128-byte runs.
__global__ __launch_bounds__(kThreads) void seq_major_vec_kernel(const u16* __restrict__ x, Lay xl,
                                                                 u16* __restrict__ y, int64_t ldy, int H, int L,
                                                                 int D) {
  const int bh = blockIdx.z, b = bh / H, h = bh % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dc = lane & 7, sg = lane >> 3;
  const int p0 = (blockIdx.x * 4 + wave) * 64 + 8 * sg, d = blockIdx.y * 64 + 8 * dc;
  if (p0 >= ldy) return;
  const u16* xb = x + b * xl.b + h * xl.h + d;
  uint32_t in[8][4];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int src = perm16(p0 + j);
    i32x4 v = {0, 0, 0, 0};
    if (src < L) v = *reinterpret_cast<const i32x4*>(xb + (int64_t)src * xl.s);
#pragma unroll
    for (int w = 0; w < 4; ++w) in[j][w] = (uint32_t)v[w];
  }
  u16* yb = y + (int64_t)bh * D * ldy + (int64_t)d * ldy + p0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {  // output row d + e: positions p0 .. p0 + 7
    const int w = e >> 1, sh = (e & 1) * 16;
    i32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = (int)(((in[2 * k][w] >> sh) & 0xffffu) | (((in[2 * k + 1][w] >> sh) & 0xffffu) << 16));
    *reinterpret_cast<i32x4*>(yb + (int64_t)e * ldy) = o;
  }
}

// ============================================================================ host dispatch
bool dtype_ok(int dt) { return dt == Q3_F32 || dt == Q3_F16 || dt == Q3_BF16; }

template <typename T, int GH, int NW>
int fwd_v3_launch(const void* q, Lay ql, const void* k, Lay kl, const void* vt, void* o, float* lse, int B, int Hq,
                  int Hkv, int Lq, int Lk, int ldvt, float scale, hipStream_t s) {
  constexpr int QT = 32 * (NW / GH);
  dim3 grid((unsigned)(B * Hq / GH), (unsigned)((Lq + QT - 1) / QT));
  attn_fwd_v3<T, GH, NW><<<grid, NW * 64, 0, s>>>((const u16*)q, ql, (const u16*)k, kl, (const u16*)vt, (u16*)o,
                                                  lse, Hq, Hkv, Lq, Lk, ldvt, scale * kLog2e);
  return (int)hipGetLastError();
}

// 8-wave workgroups (every K/V tile feeds 256 query rows) when the grid has at least two of them per
// CU; otherwise 4-wave workgroups of half the query rows, two per CU: the longest (last) query tiles
// of a causal grid bound the launch, and halving their rows halves their time.
template <typename T, int GH>
int fwd_v3(const void* q, Lay ql, const void* k, Lay kl, const void* vt, void* o, float* lse, int B, int Hq, int Hkv,
           int Lq, int Lk, int ldvt, float scale, hipStream_t s) {
  constexpr int QT8 = 32 * (8 / GH);
  if (GH <= 4 && (int64_t)(B * Hq / GH) * ((Lq + QT8 - 1) / QT8) < 512)
    return fwd_v3_launch<T, GH, 4>(q, ql, k, kl, vt, o, lse, B, Hq, Hkv, Lq, Lk, ldvt, scale, s);
  return fwd_v3_launch<T, GH, 8>(q, ql, k, kl, vt, o, lse, B, Hq, Hkv, Lq, Lk, ldvt, scale, s);
}

template <typename T, int D>
int fwd_mfma(const void* q, Lay ql, const void* k, Lay kl, const void* vt, void* o, float* lse, int B, int Hq,
             int Hkv, int Lq, int Lk, int ldvt, float scale, hipStream_t s) {
  if constexpr (D == 128) {
    // 8-wave GQA workgroups: as many heads of the group per workgroup as divide it (4, 2 or 1)
    const int grp = Hq / Hkv;
    if (grp % 4 == 0) return fwd_v3<T, 4>(q, ql, k, kl, vt, o, lse, B, Hq, Hkv, Lq, Lk, ldvt, scale, s);
    if (grp % 2 == 0) return fwd_v3<T, 2>(q, ql, k, kl, vt, o, lse, B, Hq, Hkv, Lq, Lk, ldvt, scale, s);
    return fwd_v3<T, 1>(q, ql, k, kl, vt, o, lse, B, Hq, Hkv, Lq, Lk, ldvt, scale, s);
  } else {
    // Direct-to-LDS kernel: K rows and V^T rows are 16-byte aligned (checked by the caller).
    dim3 grid((unsigned)((Lq + 127) / 128), (unsigned)(B * Hq));
    attn_fwd_v2<T, D><<<grid, kThreads, 0, s>>>((const u16*)q, ql, (const u16*)k, kl, (const u16*)vt, (u16*)o, lse,
                                                 Hq, Hkv, Lq, Lk, ldvt, scale * kLog2e);
    return (int)hipGetLastError();
  }
}

}  // namespace

// dK/dV with one query head per wave (attention_bwd.hip); Hq / Hkv must be a multiple of 4.
int q3i_attn_bwd_dkdv_v4(int dtype, const void* q, int64_t qsb, int64_t qsh, int64_t qss, const void* k,
                         const void* v, int64_t ksb, int64_t ksh, int64_t kss, const void* dout, const float* lse,
                         const float* delta, void* dk, void* dv, int B, int Hq, int Hkv, int Lq, int Lk, float scale,
                         hipStream_t s);

namespace {

template <typename T, int GH>
int bwd_dq_v3(const void* q, Lay ql, const void* k, const void* v, Lay kl, const void* kt, const void* dout,
              const float* lse, const float* delta, void* dq, int B, int Hq, int Hkv, int Lq, int Lk, int ldkt,
              float scale, hipStream_t s) {
  constexpr int QT = 32 * (8 / GH);
  dim3 g((unsigned)(B * Hq / GH), (unsigned)((Lq + QT - 1) / QT));
  attn_bwd_dq_v3<T, GH><<<g, 512, 0, s>>>((const u16*)q, ql, (const u16*)k, (const u16*)v, kl, (const u16*)kt,
                                          (const u16*)dout, lse, delta, (u16*)dq, Hq, Hkv, Lq, Lk, ldkt, scale,
                                          scale * kLog2e);
  return (int)hipGetLastError();
}

template <typename T, int D>
int bwd_mfma(const void* q, Lay ql, const void* k, const void* v, Lay kl, const void* qt, const void* kt,
             const void* dout, const void* dot, const float* lse, const float* delta, void* dq, void* dk, void* dv,
             int B, int Hq, int Hkv, int Lq, int Lk, int ldqt, int ldkt, float scale, hipStream_t s) {
  if constexpr (D == 128) {
    // dQ on 8-wave GQA workgroups (K^T copy), dK/dV with transpose reads (qt, dot unused)
    const int grp = Hq / Hkv;
    int rc;
    if (grp % 4 == 0) rc = bwd_dq_v3<T, 4>(q, ql, k, v, kl, kt, dout, lse, delta, dq, B, Hq, Hkv, Lq, Lk, ldkt, scale, s);
    else if (grp % 2 == 0)
      rc = bwd_dq_v3<T, 2>(q, ql, k, v, kl, kt, dout, lse, delta, dq, B, Hq, Hkv, Lq, Lk, ldkt, scale, s);
    else rc = bwd_dq_v3<T, 1>(q, ql, k, v, kl, kt, dout, lse, delta, dq, B, Hq, Hkv, Lq, Lk, ldkt, scale, s);
    if (rc) return rc;
    if (grp % 4 == 0)  // one query head per wave, 48-key wave tiles (attention_bwd.hip)
      return q3i_attn_bwd_dkdv_v4(T::code, q, ql.b, ql.h, ql.s, k, v, kl.b, kl.h, kl.s, dout, lse, delta, dk, dv, B,
                                  Hq, Hkv, Lq, Lk, scale, s);
    dim3 g2((unsigned)(B * Hkv), (unsigned)((Lk + 127) / 128));
    attn_bwd_dkdv_v3<T><<<g2, 256, 0, s>>>((const u16*)q, ql, (const u16*)k, (const u16*)v, kl, (const u16*)dout, lse,
                                           delta, (u16*)dk, (u16*)dv, Hq, Hkv, Lq, Lk, scale, scale * kLog2e);
    return (int)hipGetLastError();
  } else {
    // Direct-to-LDS kernels need 16-byte aligned rows of every operand (checked by the caller).
    dim3 g1((unsigned)(B * Hq), (unsigned)((Lq + 127) / 128));
    attn_bwd_dq_v2<T, D, 1><<<g1, kThreads, 0, s>>>((const u16*)q, ql, (const u16*)k, (const u16*)v, kl,
                                                     (const u16*)kt, (const u16*)dout, lse, delta, (u16*)dq, Hq, Hkv,
                                                     Lq, Lk, ldkt, scale, scale * kLog2e);
    dim3 g2((unsigned)(B * Hkv), (unsigned)((Lk + 127) / 128));
    // D = 128: one workgroup per CU either way (registers); a 3-deep ring plus the V block fits the LDS.
    attn_bwd_dkdv_v2<T, D, (D > 64 ? 1 : 2), (D > 64 ? 3 : 2)><<<g2, kThreads, 0, s>>>((const u16*)q, ql, (const u16*)k, (const u16*)v, kl,
                                                    (const u16*)qt, (const u16*)dout, (const u16*)dot, lse, delta,
                                                    (u16*)dk, (u16*)dv, Hq, Hkv, Lq, Lk, ldqt, scale, scale * kLog2e);
    return (int)hipGetLastError();
  }
}

template <typename T>
int fwd_simt(const void* q, Lay ql, const void* k, const void* v, Lay kl, void* o, float* lse, int B, int Hq, int Hkv,
             int Lq, int Lk, int D, float scale, hipStream_t s) {
  typedef typename T::storage S;
  dim3 grid((unsigned)(((int64_t)Hq * Lq + 3) / 4), 1, (unsigned)B);
  attn_fwd_simt<T><<<grid, kThreads, 0, s>>>((const S*)q, ql, (const S*)k, (const S*)v, kl, (S*)o, lse, Hq, Hkv, Lq,
                                             Lk, D, scale);
  return (int)hipGetLastError();
}

template <typename T>
int bwd_simt(const void* q, Lay ql, const void* k, const void* v, Lay kl, const void* dout, const float* lse,
             const float* delta, void* dq, void* dk, void* dv, int B, int Hq, int Hkv, int Lq, int Lk, int D,
             float scale, hipStream_t s) {
  typedef typename T::storage S;
  dim3 g1((unsigned)(((int64_t)Hq * Lq + 3) / 4), 1, (unsigned)B);
  attn_bwd_dq_simt<T><<<g1, kThreads, 0, s>>>((const S*)q, ql, (const S*)k, (const S*)v, kl, (const S*)dout, lse,
                                              delta, (S*)dq, Hq, Hkv, Lq, Lk, D, scale);
  dim3 g2((unsigned)(((int64_t)Hkv * Lk + 3) / 4), 1, (unsigned)B);
  attn_bwd_dkdv_simt<T><<<g2, kThreads, 0, s>>>((const S*)q, ql, (const S*)k, (const S*)v, kl, (const S*)dout, lse,
                                                delta, (S*)dk, (S*)dv, Hq, Hkv, Lq, Lk, D, scale);
  return (int)hipGetLastError();
}

template <typename T>
int delta_t(const void* o, const void* dout, Lay ql, float* delta, int64_t rows, int H, int L, int D, hipStream_t s) {
  typedef typename T::storage S;
  const bool vec = T::vec == 8 && (D == 128 || D == 64 || D == 32) && ql.b % 8 == 0 && ql.h % 8 == 0 &&
                   ql.s % 8 == 0 && ((uintptr_t)o & 15) == 0 && ((uintptr_t)dout & 15) == 0;
  if (vec) {
    const int lpr = D / 8, rpb = (kThreads / 64) * (64 / lpr);
    const unsigned grid = (unsigned)((rows + rpb - 1) / rpb);
    if (lpr == 16)
      attn_delta_vec_kernel<T, 16><<<grid, kThreads, 0, s>>>((const S*)o, (const S*)dout, ql, delta, rows, H, L);
    else if (lpr == 8)
      attn_delta_vec_kernel<T, 8><<<grid, kThreads, 0, s>>>((const S*)o, (const S*)dout, ql, delta, rows, H, L);
    else
      attn_delta_vec_kernel<T, 4><<<grid, kThreads, 0, s>>>((const S*)o, (const S*)dout, ql, delta, rows, H, L);
    return (int)hipGetLastError();
  }
  attn_delta_kernel<T><<<(unsigned)((rows + 3) / 4), kThreads, 0, s>>>((const S*)o, (const S*)dout, ql, delta, rows, H,
                                                                       L, D);
  return (int)hipGetLastError();
}

bool shapes_ok(int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D) {
  return B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Lq > 0 && Lk >= Lq && D > 0 && D <= 256 &&
         B * Hq < 65536 && Lk < (1 << 30);
}
bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
// The matrix-core kernels move 16-byte vectors along D: rows must be 16-byte aligned.
bool lay_ok(const void* p, Lay l) { return al16(p) && l.b % 8 == 0 && l.h % 8 == 0 && l.s % 8 == 0; }

#define Q3_ATTN_D(T, FN, ...)                                        \
  (D == 128 ? FN<T, 128>(__VA_ARGS__) : D == 64 ? FN<T, 64>(__VA_ARGS__) : FN<T, 32>(__VA_ARGS__))

}  // namespace

extern "C" {

int q3_attention_mfma_supported(int dtype, int64_t d) {
  return (dtype == Q3_BF16 || dtype == Q3_F16) && (d == 32 || d == 64 || d == 128);
}

int q3_attention_seq_major(int dtype, const void* x, int64_t sb, int64_t sh, int64_t ss, void* y, int64_t ldy,
                           int64_t B, int64_t H, int64_t L, int64_t D, hipStream_t stream) {
  Q3_REQUIRE((dtype == Q3_BF16 || dtype == Q3_F16) && x && y && B > 0 && H > 0 && L > 0 && D > 0 && ldy >= L &&
             ldy % 16 == 0 && B * H < 65536 && (D + 63) / 64 < 65536);
  if (D % 64 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 && sb % 8 == 0 && sh % 8 == 0 &&
      ss % 8 == 0) {
    dim3 grid((unsigned)((ldy + 255) / 256), (unsigned)(D / 64), (unsigned)(B * H));
    seq_major_vec_kernel<<<grid, kThreads, 0, stream>>>((const u16*)x, Lay{sb, sh, ss}, (u16*)y, ldy, (int)H,
                                                        (int)L, (int)D);
    return (int)hipGetLastError();
  }
  dim3 grid((unsigned)((ldy + 63) / 64), (unsigned)((D + 63) / 64), (unsigned)(B * H));
  seq_major_kernel<<<grid, kThreads, 0, stream>>>((const u16*)x, Lay{sb, sh, ss}, (u16*)y, ldy, (int)H, (int)L,
                                                  (int)D);
  return (int)hipGetLastError();
}

int q3_attention_fwd(int dtype, const void* q, int64_t qsb, int64_t qsh, int64_t qss, const void* k, const void* v,
                     int64_t ksb, int64_t ksh, int64_t kss, const void* vt, int64_t ldvt, void* o, float* lse,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk, int64_t D, float scale,
                     hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && q && k && o && lse && shapes_ok(B, Hq, Hkv, Lq, Lk, D));
  const Lay ql{qsb, qsh, qss}, kl{ksb, ksh, kss};
  const int b = (int)B, hq = (int)Hq, hkv = (int)Hkv, lq = (int)Lq, lk = (int)Lk;
  if (q3_attention_mfma_supported(dtype, D)) {
    Q3_REQUIRE(vt && ldvt >= Lk && ldvt % 16 == 0 && lay_ok(q, ql) && lay_ok(k, kl) && lay_ok(o, ql) && al16(vt));
    const int ld = (int)ldvt;
    if (dtype == Q3_BF16) return Q3_ATTN_D(BF16, fwd_mfma, q, ql, k, kl, vt, o, lse, b, hq, hkv, lq, lk, ld, scale, stream);
    return Q3_ATTN_D(F16, fwd_mfma, q, ql, k, kl, vt, o, lse, b, hq, hkv, lq, lk, ld, scale, stream);
  }
  Q3_REQUIRE(v);
  if (dtype == Q3_BF16) return fwd_simt<BF16>(q, ql, k, v, kl, o, lse, b, hq, hkv, lq, lk, (int)D, scale, stream);
  if (dtype == Q3_F16) return fwd_simt<F16>(q, ql, k, v, kl, o, lse, b, hq, hkv, lq, lk, (int)D, scale, stream);
  return fwd_simt<F32>(q, ql, k, v, kl, o, lse, b, hq, hkv, lq, lk, (int)D, scale, stream);
}

int q3_attention_bwd(int dtype, const void* q, int64_t qsb, int64_t qsh, int64_t qss, const void* k, const void* v,
                     int64_t ksb, int64_t ksh, int64_t kss, const void* o, const void* dout, const float* lse,
                     const void* qt, int64_t ldqt, const void* kt, int64_t ldkt, const void* dot, float* delta,
                     void* dq, void* dk, void* dv, int64_t B, int64_t Hq, int64_t Hkv, int64_t Lq, int64_t Lk,
                     int64_t D, float scale, hipStream_t stream) {
  Q3_REQUIRE(dtype_ok(dtype) && q && k && v && o && dout && lse && delta && dq && dk && dv &&
             shapes_ok(B, Hq, Hkv, Lq, Lk, D));
  const Lay ql{qsb, qsh, qss}, kl{ksb, ksh, kss};
  const int b = (int)B, hq = (int)Hq, hkv = (int)Hkv, lq = (int)Lq, lk = (int)Lk, d = (int)D;
  int rc;
  if (dtype == Q3_BF16) rc = delta_t<BF16>(o, dout, ql, delta, B * Hq * Lq, hq, lq, d, stream);
  else if (dtype == Q3_F16) rc = delta_t<F16>(o, dout, ql, delta, B * Hq * Lq, hq, lq, d, stream);
  else rc = delta_t<F32>(o, dout, ql, delta, B * Hq * Lq, hq, lq, d, stream);
  if (rc) return rc;
  if (q3_attention_mfma_supported(dtype, D)) {
    // D = 128 reads Q and dO transposed straight from LDS: qt / dot are not needed (may be null)
    const bool need_qt = D != 128;
    Q3_REQUIRE(kt && ldkt >= Lk && ldkt % 16 == 0 && lay_ok(q, ql) && lay_ok(dout, ql) && lay_ok(dq, ql) &&
               lay_ok(k, kl) && lay_ok(v, kl) && lay_ok(dk, kl) && lay_ok(dv, kl) && al16(kt));
    Q3_REQUIRE(!need_qt || (qt && dot && ldqt >= Lq && ldqt % 16 == 0 && al16(qt) && al16(dot)));
    const int lq8 = (int)ldqt, lk8 = (int)ldkt;
    if (dtype == Q3_BF16)
      return Q3_ATTN_D(BF16, bwd_mfma, q, ql, k, v, kl, qt, kt, dout, dot, lse, delta, dq, dk, dv, b, hq, hkv, lq, lk,
                       lq8, lk8, scale, stream);
    return Q3_ATTN_D(F16, bwd_mfma, q, ql, k, v, kl, qt, kt, dout, dot, lse, delta, dq, dk, dv, b, hq, hkv, lq, lk,
                     lq8, lk8, scale, stream);
  }
  if (dtype == Q3_BF16)
    return bwd_simt<BF16>(q, ql, k, v, kl, dout, lse, delta, dq, dk, dv, b, hq, hkv, lq, lk, d, scale, stream);
  if (dtype == Q3_F16)
    return bwd_simt<F16>(q, ql, k, v, kl, dout, lse, delta, dq, dk, dv, b, hq, hkv, lq, lk, d, scale, stream);
  return bwd_simt<F32>(q, ql, k, v, kl, dout, lse, delta, dq, dk, dv, b, hq, hkv, lq, lk, d, scale, stream);
}

}  // extern "C"

// Causal GQA attention backward at head_dim 128: the dK/dV kernel with one query head per wave.
//
// Workgroup = the 4 query heads of one KV head (4 waves, one per SIMD, ratio Hq/Hkv a multiple of 4:
// wave w takes heads w, w + 4, ...), all on the same 48 keys.  Each wave holds the K and V fragments
// of the 48 keys in registers (B operands) and its dK^T / dV^T accumulators (48 keys x 128 dims
// each), and streams its own head's Q / dO / lse / delta tiles of 32 queries through a private
// 2-stage direct-to-LDS ring -- no workgroup barrier inside the loop.  Per tile:
//   S = Q K^T, dP = dO V^T - delta (Q / dO row fragments from LDS),
//   P = exp2(S scale log2e - lse log2e), dS = P dP,
//   dV^T += dO^T P, dK^T += Q^T dS (dO^T / Q^T by LDS transpose reads of the same tiles).
// 48 keys per wave give every LDS fragment three MFMAs (the 32-key wave tile of attn_bwd_dkdv_v3 gives
// two): 2/3 of the LDS traffic per MFMA.  (64 keys do not fit: K/V fragments + the S / dP tiles
// exceed the 256 VGPRs beside the 256 AGPRs of the accumulators.)  The 4 heads' partial dK / dV fold through LDS in fixed
// order at the end (deterministic, no atomics).  Causal balance: one key tile per workgroup, the
// tiles with the most queries first (a longest-first list schedule over the CUs).
#include <type_traits>

#include "common.h"

namespace {

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((address_space(3))) void* lds_vp;
constexpr float kLog2e = 1.4426950408889634f;

constexpr int kD = 128, kC = 3, kBN = 16 * kC, kBM = 32, kST = 2;  // kC key sub-tiles of 16 per wave
constexpr int kTB = kBM * kD * 2;                 // one [32 x 128] 16-bit tile: 8 KB
constexpr int kStage = 2 * kTB + 2 * kBM * 4;     // Q, dO, lse, delta
constexpr int kWaveLds = kST * kStage;            // private ring of one wave
constexpr int kRed = kBN * kD * 4;                // one wave's fp32 dK (or dV) block
static_assert(4 * kRed <= 4 * kWaveLds, "the fold reuses the rings");

Q3_DEV i32x4 ld16(const u16* p) { return *reinterpret_cast<const i32x4*>(p); }
Q3_DEV bf16x8_t as_frag(i32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }
// 8 bytes by the gfx950 transpose read: within each 16-lane group, lane j receives element j % 4 of
// the 8-byte pieces addressed by lanes j / 4 + 4 k, k = 0..3.
Q3_DEV i32x2 ldtr(const char* p) {
  return __builtin_bit_cast(i32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)p));
}
// 16-byte chunk swizzle of the 256-byte query rows: conflict-free row reads (16 rows of one chunk
// column) and distinct 32-byte bank groups for the 8 rows of each half-wave transpose read.
Q3_DEV int qswz(int r) { return 2 * ((r & 3) | (((r >> 3) & 1) << 2)) + ((r >> 4) & 1); }

// dK^T / dV^T accumulation, D(AGPR) += A B: the 64 accumulator quads of each stay in AGPRs (the
// S / dP products of the same loop are VGPR-form builtins), so the register allocator never moves
// them.  The leading s_nop covers the VALU-write -> MFMA-read distance of the packed P / dS operands
// (issued while the previous MFMA occupies the pipe).
template <typename T> Q3_DEV void mfma_acc(f32x4& acc, i32x4 a, i32x4 b);
template <> Q3_DEV void mfma_acc<BF16>(f32x4& acc, i32x4 a, i32x4 b) {
  asm("s_nop 4\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
template <> Q3_DEV void mfma_acc<F16>(f32x4& acc, i32x4 a, i32x4 b) {
  asm("s_nop 4\n\tv_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// A zero accumulator quad produced in AGPRs (0 x 0 + 0 on the matrix core), so every definition and
// use of the accumulators is AGPR-constrained and the loop-carried values never pass through VGPRs.
Q3_DEV f32x4 agpr_zero() {
  f32x4 z;
  // the zero operand is written by a VALU move just before: the nop covers that distance
  asm volatile("s_nop 4\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %1, 0" : "=a"(z) : "v"(i32x4{0, 0, 0, 0}));
  return z;
}
// Wait states after the last asm MFMA before its accumulators are read (the compiler does not track
// the latency of inline-asm MFMAs): 4 x 8 >= the 8-pass 16x16x32 write latency.
Q3_DEV void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

Q3_DEV void wait_vm(int n) {  // vmcnt(n) for n in {0, 17}; lgkm / exp counters untouched
  if (n >= 17) __builtin_amdgcn_s_waitcnt((17 & 15) | ((17 >> 4) << 14) | (7 << 4) | (0xF << 8));
  else __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (0xF << 8));
}

template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_bwd_dkdv_v4(
    const u16* __restrict__ Q, int64_t qsb, int64_t qsh, int64_t qss, const u16* __restrict__ K,
    const u16* __restrict__ V, int64_t ksb, int64_t ksh, int64_t kss, const u16* __restrict__ dO,
    const float* __restrict__ LSE, const float* __restrict__ Delta, u16* __restrict__ dK, u16* __restrict__ dV,
    int Hq, int Hkv, int Lq, int Lk, int ntiles, float scale, float scale2) {
  __shared__ __attribute__((aligned(1024))) char lds[4 * kWaveLds];
  // One key tile per workgroup, launched in order of decreasing causal work: workgroup i takes key
  // tile i / (B Hkv) of (batch, KV head) i % (B Hkv), so the dispatcher, which hands out workgroups in
  // order as CUs free up, runs a longest-first list schedule (the tiles of one KV head are B Hkv
  // workgroups apart: with B Hkv a multiple of 8 they share an XCD and its L2 copy of Q / dO).
  const int nbk = (int)(gridDim.x / ntiles);
  const int bk = (int)(blockIdx.x % nbk), b = bk / Hkv, hk = bk % Hkv, ratio = Hq / Hkv, hpw = ratio / 4;
  const int tid = threadIdx.x, lane = tid & 63, G = lane >> 4, r16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int off = Lk - Lq;
  char* wl = lds + wave * kWaveLds;

  // row reads: query row qrow0 (+ 4 t), chunk 4 ks + G; transpose reads: group G, lane i of read h
  // addresses query row 8 G + 4 h + i / 4, bytes 32 dt + 8 (i % 4)
  const int qrow0 = 8 * (r16 >> 2) + (r16 & 3);
  int roff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) roff[ks] = qrow0 * 256 + (((4 * ks + G) ^ qswz(qrow0)) << 4);
  auto tr_addr = [&](int h, int dt) {
    const int row = 8 * G + 4 * h + (r16 >> 2);
    const int byte = 32 * dt + 8 * (r16 & 3);
    return row * 256 + ((((byte >> 4) ^ qswz(row)) << 4) | (byte & 15));
  };

  const int64_t kvbase = (int64_t)b * ksb + (int64_t)hk * ksh;

  {
    const int kt = (int)(blockIdx.x / nbk);
    const int k0 = kt * kBN;

    // K / V B operands: lane (G, r16) holds key k0 + 16 c + r16, dims 32 ks + 8 G .. + 7
    bf16x8_t kf[kC][4], vf[kC][4];
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      const int64_t row = kvbase + (int64_t)min(k0 + 16 * c + r16, Lk - 1) * kss;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        kf[c][ks] = as_frag(ld16(K + row + 32 * ks + 8 * G));
        vf[c][ks] = as_frag(ld16(V + row + 32 * ks + 8 * G));
      }
    }
    f32x4 dk[8][kC], dv[8][kC];
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int c = 0; c < kC; ++c) {
        dk[d][c] = agpr_zero();
        dv[d][c] = agpr_zero();
      }

    mfma_drain();  // the zeroed accumulators are written before the first asm MFMA reads them
    const int qstart = max(0, k0 - off) / kBM * kBM;
    const int nq = qstart < Lq ? (Lq - qstart + kBM - 1) / kBM : 0;
    const int total = hpw * nq;

    auto issue = [&](int u) {  // 8 + 8 wave loads of 4 rows x 256 B (Q, dO), one of lse / delta
      const int hh = u / nq, q0 = qstart + (u % nq) * kBM;
      const int h = hk * ratio + wave + 4 * hh;
      const int64_t bh = (int64_t)b * Hq + h;
      // wave-uniform bases (SGPRs) + 32-bit per-lane byte offsets
      const char* Qb = reinterpret_cast<const char*>(Q + b * qsb + h * qsh);
      const char* dOb = reinterpret_cast<const char*>(dO + b * qsb + h * qsh);
      char* base = wl + (u % kST) * kStage;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 4 * i + (lane >> 4);
        const int c = (lane & 15) ^ qswz(r);
        const uint32_t src = (uint32_t)(min(q0 + r, Lq - 1) * (int)qss + c * 8) * 2u;
        __builtin_amdgcn_global_load_lds(Qb + src, (lds_vp)(base + i * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(dOb + src, (lds_vp)(base + kTB + i * 1024), 16, 0, 0);
      }
      const uint32_t qq = (uint32_t)min(q0 + (lane & 31), Lq - 1) * 4u;
      const char* side = reinterpret_cast<const char*>((lane < 32 ? LSE : Delta) + bh * Lq);
      __builtin_amdgcn_global_load_lds(side + qq, (lds_vp)(base + 2 * kTB), 4, 0, 0);
    };

    if (total > 0) issue(0);
#pragma nounroll
    for (int u = 0; u < total; ++u) {
      // this wave's reads of the stage about to be refilled (tile u - 1) are complete, then the
      // refill with tile u + 1, then tile u landed (its 17 loads older than the refill's 17)
      __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
      asm volatile("" ::: "memory");
      if (u + 1 < total) {
        issue(u + 1);
        wait_vm(17);
      } else {
        wait_vm(0);
      }
      asm volatile("" ::: "memory");
      const int q0 = qstart + (u % nq) * kBM;
      if (min(q0 + kBM - 1, Lq - 1) + off < k0) continue;  // no query of the tile sees these keys
      // Tiles that cross the diagonal or the end of the queries mask P (a uniform branch around the
      // P computation only: two copies of the whole tile body made the register allocator copy the
      // accumulators between them).
      const bool masked = !(k0 + kBN - 1 <= q0 + off && q0 + kBM - 1 < Lq);
      {
        const char* qb = wl + (u % kST) * kStage;
        const char* db = qb + kTB;
        const float* side = reinterpret_cast<const float*>(qb + 2 * kTB);
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(side + 8 * G);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(side + 8 * G + 4);
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(side + kBM + 8 * G);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(side + kBM + 8 * G + 4);

        // S and dP (dP starts from -delta, its row constant, so the products leave dP - delta);
        // MFMA row r16 of query sub-tile t reads query 8 (r16 / 4) + 4 t + r16 % 4, so lane group G
        // holds queries 8 G .. 8 G + 7 of each key: P and dS pack straight into the B operands.

        float nl[2][4];
  #pragma unroll
        for (int i = 0; i < 4; ++i) {
          nl[0][i] = -l0[i] * kLog2e;
          nl[1][i] = -l1[i] * kLog2e;
        }
        // Fragment reads run one k-step ahead of their MFMAs, behind scheduling fences (without the
        // fences the scheduler hoists every LDS read of the tile and runs out of registers).
        f32x4 s[2][kC], dp[2][kC];
        i32x4 qa[2][2], da[2][2];
        auto rows = [&](int ks, int buf) {
  #pragma unroll
          for (int t = 0; t < 2; ++t) {
            qa[buf][t] = *reinterpret_cast<const i32x4*>(qb + roff[ks] + 4 * t * 256);
            da[buf][t] = *reinterpret_cast<const i32x4*>(db + roff[ks] + 4 * t * 256);
          }
        };
        rows(0, 0);
  #pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          __builtin_amdgcn_sched_barrier(0);
          if (ks < 3) rows(ks + 1, (ks + 1) & 1);
          const int cb = ks & 1;
  #pragma unroll
          for (int t = 0; t < 2; ++t)
  #pragma unroll
            for (int c = 0; c < kC; ++c) {
              s[t][c] = mfma_16x16x32<T>(as_frag(qa[cb][t]), kf[c][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[t][c]);
              dp[t][c] = mfma_16x16x32<T>(as_frag(da[cb][t]), vf[c][ks], ks == 0 ? -(t ? d1 : d0) : dp[t][c]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        i32x4 pp[kC], dd[kC];
        auto probs = [&](auto mask_c) {
          constexpr bool MASK = decltype(mask_c)::value;
  #pragma unroll
          for (int c = 0; c < kC; ++c) {
            float pv[8], dsv[8];
  #pragma unroll
            for (int t = 0; t < 2; ++t)
  #pragma unroll
              for (int i = 0; i < 4; ++i) {
                float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][c][i], scale2, nl[t][i]));
                if constexpr (MASK) {
                  const int q = q0 + 8 * G + 4 * t + i;
                  p = (k0 + 16 * c + r16 <= q + off && q < Lq) ? p : 0.f;
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
        };
        if (masked) probs(std::true_type{});
        else probs(std::false_type{});
        i32x4 aq[2], ad[2];
        auto trs = [&](int dt, int buf) {
          const i32x2 q0v = ldtr(qb + tr_addr(0, dt)), q1v = ldtr(qb + tr_addr(1, dt));
          const i32x2 d0v = ldtr(db + tr_addr(0, dt)), d1v = ldtr(db + tr_addr(1, dt));
          aq[buf] = i32x4{q0v[0], q0v[1], q1v[0], q1v[1]};
          ad[buf] = i32x4{d0v[0], d0v[1], d1v[0], d1v[1]};
        };
        trs(0, 0);
  #pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          __builtin_amdgcn_sched_barrier(0);
          if (dt < 7) trs(dt + 1, (dt + 1) & 1);
          const int cb = dt & 1;
  #pragma unroll
          for (int c = 0; c < kC; ++c) {
            mfma_acc<T>(dv[dt][c], ad[cb], pp[c]);
            mfma_acc<T>(dk[dt][c], aq[cb], dd[c]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    mfma_drain();
    // Fold the 4 waves' partial dK^T / dV^T (lane holds [d = 16 dt + 4 G + i][key = k0 + 16 c + r16])
    // in wave order through LDS (the rings are drained: every issued tile was waited for).
    auto fold = [&](f32x4 (&acc)[8][kC], u16* out, float mul) {
      __syncthreads();
      f32x4* mine = reinterpret_cast<f32x4*>(lds + wave * kRed);
      // stored straight from the AGPRs (a C++ read of the accumulators would make the register
      // allocator keep them in VGPRs for the whole loop)
      const uint32_t mbase = (uint32_t)(uintptr_t)(mine + lane);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int c = 0; c < kC; ++c)
          asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(mbase), "a"(acc[dt][c]), "i"((dt * kC + c) * 64 * 16)
                       : "memory");
      __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 2 * kC; ++j) {
        const int idx = (wave * 2 * kC + j) * 64 + lane;  // f32x4 slot: (dt, c) = idx / 64, source lane idx % 64
        f32x4 sum = reinterpret_cast<const f32x4*>(lds)[idx];
#pragma unroll
        for (int w = 1; w < 4; ++w) sum += reinterpret_cast<const f32x4*>(lds + w * kRed)[idx];
        const int dc = idx >> 6, dt = dc / kC, c = dc % kC, sl = idx & 63;
        const int key = k0 + 16 * c + (sl & 15), d = 16 * dt + 4 * (sl >> 4);
        if (key < Lk) {
          i32x2 wv;
          wv[0] = (int)pack2<T>(sum[0] * mul, sum[1] * mul);
          wv[1] = (int)pack2<T>(sum[2] * mul, sum[3] * mul);
          *reinterpret_cast<i32x2*>(out + kvbase + (int64_t)key * kss + d) = wv;
        }
      }
    };
    fold(dk, dK, scale);
    fold(dv, dV, 1.f);
  }
}

}  // namespace

// Launcher used by q3_attention_bwd (attention.hip) for D = 128 when Hq / Hkv is a multiple of 4.
// Strides are element strides (batch, head, position) of [B, H, L, 128] operands with 16-byte rows.
int q3i_attn_bwd_dkdv_v4(int dtype, const void* q, int64_t qsb, int64_t qsh, int64_t qss, const void* k,
                         const void* v, int64_t ksb, int64_t ksh, int64_t kss, const void* dout, const float* lse,
                         const float* delta, void* dk, void* dv, int B, int Hq, int Hkv, int Lq, int Lk, float scale,
                         hipStream_t s) {
  if ((Hq / Hkv) % 4 != 0) return Q3_ERR_INVALID;
  const int ntiles = (Lk + kBN - 1) / kBN;
  const dim3 g((unsigned)(B * Hkv * ntiles));
  if (dtype == Q3_BF16)
    attn_bwd_dkdv_v4<BF16><<<g, 256, 0, s>>>((const u16*)q, qsb, qsh, qss, (const u16*)k, (const u16*)v, ksb, ksh,
                                             kss, (const u16*)dout, lse, delta, (u16*)dk, (u16*)dv, Hq, Hkv, Lq, Lk,
                                             ntiles, scale, scale * kLog2e);
  else
    attn_bwd_dkdv_v4<F16><<<g, 256, 0, s>>>((const u16*)q, qsb, qsh, qss, (const u16*)k, (const u16*)v, ksb, ksh,
                                            kss, (const u16*)dout, lse, delta, (u16*)dk, (u16*)dv, Hq, Hkv, Lq, Lk,
                                            ntiles, scale, scale * kLog2e);
  return (int)hipGetLastError();
}

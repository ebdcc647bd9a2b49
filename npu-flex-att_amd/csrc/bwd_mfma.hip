// Flash-attention backward for fp16/bf16 on gfx950 MFMA: the dQ kernel and
// the dK/dV kernel.  Delta = rowsum(O * dO) comes from the pre-kernel in
// delta.hip.
//
// Semantics: npu_flash_attention.py:298-402 (flash_attn_bwd_dq_kernel) and
// :407-560 (flash_attn_bwd_dkdv_kernel): P is recomputed from the forward LSE,
// dP = dO V^T, dS = P (dP - Delta) scale (1 - tanh^2), dQ = dS K,
// dK = dS^T Q, dV = P^T dO; P and dS are rounded to the input dtype before
// their MFMAs, as the reference does before tl.dot.  Two deliberate
// differences: the ALiBi bias is part of the recomputed P (the reference's
// backward kernels take no ALiBi argument), and dK/dV are accumulated over the
// G query heads of a group in fp32 inside the kernel (the reference writes
// per-query-head partials and sums them in the input dtype,
// npu_flash_attention.py:734-737).
//
// dQ: one workgroup = 4 waves = 128 query rows of one (b, hq); per 64-row KV
//     tile each wave forms S^T = K Q^T and dP^T = V dO^T (lane = query row),
//     then dQ^T += K^T dS^T with K^T read by the LDS transpose read.
// dK/dV: one workgroup = 4 waves = 128 KV rows of one (b, hkv); K and V rows
//     live in registers; the workgroup walks the G query heads of the group
//     and their 64-row query tiles, forming S = Q K^T and dP = dO V^T
//     (lane = KV row), then dV^T += dO^T P and dK^T += Q^T dS with dO^T and
//     Q^T read by the LDS transpose read.
// Both kernels are deterministic: every output element is owned by one lane
// and accumulated in a fixed order.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

template <int D>
struct BwdCfg {
  static constexpr int NW = 4;
  static constexpr int KC = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int P = D + 8;
  static constexpr int CPR = D / 8;
  // dQ kernel
  static constexpr int BM = 32 * NW;
  static constexpr int BN = 64;
  static constexpr int CPT = BN * CPR / (NW * 64);
  // dK/dV kernel
  static constexpr int BNK = 32 * NW;
  // query rows per dK/dV tile: 128 at D = 32, where a 64-row tile carries too
  // little MFMA work per barrier (0.53 -> 0.47 ms at bf16 B=2 Hq=32 Hkv=8
  // S=4096 causal)
  static constexpr int BMQ = D == 32 ? 128 : 64;
  static constexpr int CPTQ = BMQ * CPR / (NW * 64);
  static constexpr bool PREFETCH = D <= 128;
  // D = 256: dV and dK in two passes over the query tiles (S recomputed), so
  // that the K / V rows and both accumulator sets never share the registers
  static constexpr bool SPLIT = D == 256;
  // waves per SIMD the register budget targets: two workgroups per CU for
  // D <= 64 (their VALU work then overlaps the other workgroup's MFMAs)
  static constexpr int WPE = D <= 64 ? 2 : 1;
  // the D = 32 dQ kernel fits three waves per SIMD (at most 163 VGPRs):
  // 0.243 against 0.287 ms at bf16 B=2 Hq=32 Hkv=8 S=4096 causal (dK/dV does
  // not change at three)
  static constexpr int WPE_DQ = D == 32 ? 3 : WPE;
};

// ---------------------------------------------------------------- dQ kernel --
template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BwdCfg<D>::WPE_DQ, BwdCfg<D>::WPE_DQ)))
void bwd_dq_mfma_kernel(BwdArgs a) {
  using C = BwdCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(16))) T sK[C::BN * C::P];
  __shared__ __attribute__((aligned(16))) T sV[C::BN * C::P];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar branches)
  const int h = lane >> 5, l32 = lane & 31;

  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.ntiles - 1 - (w % a.ntiles);
  const int bh = w / a.ntiles;
  const int hq = bh % p.Hq, b = bh / p.Hq;
  const int hk = hq / p.G;
  const int m0 = qt * C::BM;
  const int mw = m0 + wave * 32;
  const int my_m = mw + l32;

  const T* qp = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh;
  const T* dop = (const T*)a.dout.data + b * a.dout.sb + hq * a.dout.sh;
  const T* kp = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const T* vp = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh;

  V8 qf[C::KC], dof[C::KC];
  {
    const int r = min(my_m, p.Sq - 1);
    const T* sq = qp + (int64_t)r * a.q.ss + 8 * h;
    const T* sd = dop + (int64_t)r * a.dout.ss + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      i32x4 x = ld_global16(sq + 16 * kc), y = ld_global16(sd + 16 * kc);
      if (my_m >= p.Sq) { x = i32x4{0, 0, 0, 0}; y = i32x4{0, 0, 0, 0}; }
      qf[kc] = as_v8<V8>(x);
      dof[kc] = as_v8<V8>(y);
    }
  }
  // log2-domain LSE; +inf makes P exactly 0 for fully-masked or padding rows.
  float lse2 = kPosInf, dl = 0.f;
  if (my_m < p.Sq) {
    const int64_t ri = (int64_t)(b * p.Hq + hq) * p.Sq + my_m;
    const float l = a.lse[ri];
    lse2 = (l == kNegInf) ? kPosInf : l * kLog2e;
    dl = a.delta[ri];
  }

  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + C::BM);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
  // document masks: this lane's bounds, the KV range of the workgroup's and
  // of this wave's rows
  int dlo, dhi, wlo = 0, whi = 0x7fffffff;
  doc_bounds(p, b, min(my_m, p.Sq - 1), dlo, dhi);
  if (p.doc) {
    int l0, h0, l1, h1;
    doc_bounds(p, b, min(m0, p.Sq - 1), l0, h0);
    doc_bounds(p, b, min(m0 + C::BM, p.Sq) - 1, l1, h1);
    kv_lo = max(kv_lo, l0);
    kv_hi = min(kv_hi, h1);
    doc_bounds(p, b, min(mw, p.Sq - 1), wlo, h0);
    doc_bounds(p, b, min(mw + 31, p.Sq - 1), l1, whi);
  }
  const int t_lo = kv_lo / C::BN;
  const int t_hi = (kv_hi + C::BN - 1) / C::BN;

  i32x4 rk[C::CPT], rv[C::CPT];
  auto gload = [&](int t) {
    const int n0 = t * C::BN;
#pragma unroll
    for (int e = 0; e < C::CPT; ++e) {
      const int c = tid + e * C::NW * 64;
      const int row = c / C::CPR, col = (c % C::CPR) * 8;
      const int n = n0 + row;
      const int nc = min(n, p.Skv - 1);
      // rows past Skv load row Skv - 1: their P is masked to 0, so they add
      // nothing, and nothing reads the loaded registers before lstore (a
      // select here would wait for the prefetch at once)
      rk[e] = ld_global16(kp + (int64_t)nc * a.k.ss + col);
      rv[e] = ld_global16(vp + (int64_t)nc * a.v.ss + col);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int e = 0; e < C::CPT; ++e) {
      const int c = tid + e * C::NW * 64;
      const int row = c / C::CPR, col = (c % C::CPR) * 8;
      *(i32x4*)&sK[row * C::P + col] = rk[e];
      *(i32x4*)&sV[row * C::P + col] = rv[e];
    }
  };

  f32x16 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x16{};
  const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;

  if (C::PREFETCH && t_lo < t_hi) gload(t_lo);
  for (int t = t_lo; t < t_hi; ++t) {
    if (t > t_lo) __syncthreads();
    if (!C::PREFETCH) gload(t);
    lstore();
    __syncthreads();
    if (C::PREFETCH && t + 1 < t_hi) gload(t + 1);

    const int n0 = t * C::BN;
    const bool skip = (p.causal && n0 > mw + 31) || (p.window > 0 && mw - (n0 + C::BN - 1) > p.window) ||
                      n0 >= whi || n0 + C::BN <= wlo ||
                      !__builtin_amdgcn_readfirstlane(block_on(p, b, hq, min(mw, p.Sq - 1), n0));
    if (skip) continue;
    const bool full = (n0 + C::BN <= p.Skv) && (!p.causal || n0 + C::BN - 1 <= mw) &&
                      (p.window == 0 || mw + 31 - n0 <= p.window) && !p.doc;

    f32x16 s[2], dp[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      s[bb] = f32x16{};
      dp[bb] = f32x16{};
      const T* kr = sK + (32 * bb + l32) * C::P + 8 * h;
      const T* vr = sV + (32 * bb + l32) * C::P + 8 * h;
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc) {
        s[bb] = M::mma(as_v8<V8>(lds_read16(kr + 16 * kc)), qf[kc], s[bb]);
        dp[bb] = M::mma(as_v8<V8>(lds_read16(vr + 16 * kc)), dof[kc], dp[bb]);
      }
    }
    const float fb = (float)(my_m - n0 - 4 * h);  // i - j = fb - (32 bb + 8 (r / 4) + r % 4), exact
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = n0 + 32 * bb + 8 * (r >> 2) + 4 * h + (r & 3);
        float tv = 0.f;
        const float y = score_log2_d<SOFTCAP, ALIBI>(s[bb][r], p, slope_log2,
                                                     fb - (float)(32 * bb + 8 * (r >> 2) + (r & 3)), tv);
        float pr = fast_exp2(y - lse2);
        if (!full && (!allowed(p, my_m, j) || j < dlo || j >= dhi)) pr = 0.f;
        float ds = pr * (dp[bb][r] - dl) * p.scale;
        if constexpr (SOFTCAP) ds *= (1.0f - tv * tv);
        s[bb][r] = ds;
      }
    }
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const V8 dsb = pack8<T>(s[bb], 8 * c);
        const int row = 32 * bb + 16 * c + 4 * h + ((lane & 15) >> 2);
        const T* kr = sK + row * C::P + tr_col;
#pragma unroll
        for (int db = 0; db < C::DB; ++db) {
          const i16x4 lo = lds_read_tr4(kr + 32 * db);
          const i16x4 hi = lds_read_tr4(kr + 8 * C::P + 32 * db);
          acc[db] = M::mma(cat_tr<V8>(lo, hi), dsb, acc[db]);
        }
      }
    }
  }

  if (my_m < p.Sq) {
    T* op = (T*)a.dq.data + b * a.dq.sb + hq * a.dq.sh + (int64_t)my_m * a.dq.ss + 4 * h;
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st_global8(op + 32 * db + 8 * i,
                   pack4<T>(acc[db][4 * i], acc[db][4 * i + 1], acc[db][4 * i + 2], acc[db][4 * i + 3]));
    }
  }
}

// -------------------------------------------------------------- dK/dV kernel --
template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BwdCfg<D>::WPE, BwdCfg<D>::WPE)))
void bwd_dkdv_mfma_kernel(BwdArgs a) {
  using C = BwdCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(16))) T sQ[C::BMQ * C::P];
  __shared__ __attribute__((aligned(16))) T sO[C::BMQ * C::P];  // dO tile
  __shared__ __attribute__((aligned(16))) float sL[C::BMQ];      // log2-domain LSE
  __shared__ __attribute__((aligned(16))) float sDl[C::BMQ];     // Delta

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar branches)
  const int h = lane >> 5, l32 = lane & 31;

  // (b, hkv, kv-tile); under a causal mask the first KV tiles carry the most
  // query rows and are dispatched first.
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int kt = w % a.ntiles;
  const int bh = w / a.ntiles;
  const int hk = bh % p.Hkv, b = bh / p.Hkv;
  const int n0 = kt * C::BNK;
  const int nw = n0 + wave * 32;
  const int my_n = nw + l32;

  // K / V rows of this lane as MFMA B operands (k = 8 consecutive d).
  const int rkv = min(my_n, p.Skv - 1);
  auto load_rows = [&](const View& t, V8 (&f)[C::KC]) {
    const T* src = (const T*)t.data + b * t.sb + hk * t.sh + (int64_t)rkv * t.ss + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      i32x4 x = ld_global16(src + 16 * kc);
      if (my_n >= p.Skv) x = i32x4{0, 0, 0, 0};
      f[kc] = as_v8<V8>(x);
    }
  };

  int q_lo = p.causal ? n0 : 0;
  int q_hi = p.Sq;
  if (p.window > 0) q_hi = min(q_hi, n0 + C::BNK + p.window);
  // interval masks: the query range of this lane's KV row (column bounds),
  // of the workgroup's and of this wave's KV rows
  int dlo, dhi, wlo = 0, whi = 0x7fffffff;
  col_bounds(p, b, min(my_n, p.Skv - 1), dlo, dhi);
  if (p.docc) {
    int l0, h0, l1, h1;
    col_bounds(p, b, min(n0, p.Skv - 1), l0, h0);
    col_bounds(p, b, min(n0 + C::BNK, p.Skv) - 1, l1, h1);
    q_lo = max(q_lo, l0);
    q_hi = min(q_hi, h1);
    col_bounds(p, b, min(nw, p.Skv - 1), wlo, h0);
    col_bounds(p, b, min(nw + 31, p.Skv - 1), l1, whi);
  }
  const int qt_lo = q_lo / C::BMQ;
  const int qt_hi = (q_hi + C::BMQ - 1) / C::BMQ;
  const int nq = max(0, qt_hi - qt_lo);
  const int iters = nq * p.G;

  i32x4 rq[C::CPTQ], ro[C::CPTQ];
  float rl = 0.f, rd = 0.f;
  auto gload = [&](int it) {
    const int g = it / nq;
    const int hq = hk * p.G + g;
    const int m0 = (qt_lo + it % nq) * C::BMQ;
    const T* qp = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh;
    const T* dop = (const T*)a.dout.data + b * a.dout.sb + hq * a.dout.sh;
#pragma unroll
    for (int e = 0; e < C::CPTQ; ++e) {
      const int c = tid + e * C::NW * 64;
      const int row = c / C::CPR, col = (c % C::CPR) * 8;
      const int m = m0 + row;
      const int mc = min(m, p.Sq - 1);
      // rows past Sq load row Sq - 1: their LSE is +inf (P = 0), so they add
      // nothing, and nothing reads the loaded registers before lstore (a
      // select here would wait for the prefetch at once)
      rq[e] = ld_global16(qp + (int64_t)mc * a.q.ss + col);
      ro[e] = ld_global16(dop + (int64_t)mc * a.dout.ss + col);
    }
    if (tid < C::BMQ) {
      const int m = m0 + tid;
      rl = kNegInf;  // raw LSE, converted in lstore (-inf -> +inf: P = 0)
      rd = 0.f;
      if (m < p.Sq) {
        const int64_t ri = (int64_t)(b * p.Hq + hq) * p.Sq + m;
        rl = a.lse[ri];
        rd = a.delta[ri];
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int e = 0; e < C::CPTQ; ++e) {
      const int c = tid + e * C::NW * 64;
      const int row = c / C::CPR, col = (c % C::CPR) * 8;
      *(i32x4*)&sQ[row * C::P + col] = rq[e];
      *(i32x4*)&sO[row * C::P + col] = ro[e];
    }
    if (tid < C::BMQ) {
      sL[tid] = (rl == kNegInf) ? kPosInf : rl * kLog2e;  // log2 units; +inf makes P exactly 0
      sDl[tid] = rd;
    }
  };

  V8 kf[C::KC], vf[C::KC];
  f32x16 adk[C::DB], adv[C::DB];

  // One pass over the query tiles of the group, accumulating dV^T (DV) and/or
  // dK^T (DK).  A dV-only pass needs neither dP nor the V rows.
  auto run = [&](auto dv_c, auto dk_c) {
    constexpr bool DV = decltype(dv_c)::value, DK = decltype(dk_c)::value;
    if (C::PREFETCH && iters > 0) gload(0);
    for (int it = 0; it < iters; ++it) {
      if (it > 0) __syncthreads();
      if (!C::PREFETCH) gload(it);
      lstore();
      __syncthreads();
      if (C::PREFETCH && it + 1 < iters) gload(it + 1);

      const int g = it / nq;
      const int hq = hk * p.G + g;
      const int mt = (qt_lo + it % nq) * C::BMQ;
      const bool skip = (p.causal && mt + C::BMQ - 1 < nw) || (p.window > 0 && mt - (nw + 31) > p.window) ||
                        mt >= whi || mt + C::BMQ <= wlo ||
                        !__builtin_amdgcn_readfirstlane(block_on(p, b, hq, min(mt, p.Sq - 1), min(nw, p.Skv - 1)));
      if (skip) continue;
      const bool full = (!p.causal || mt >= nw + 31) && (p.window == 0 || mt + C::BMQ - 1 - nw <= p.window) &&
                        !p.doc;
      const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;
      const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      const float fq = (float)(mt + 4 * h - my_n);

#pragma unroll
      for (int mb = 0; mb < C::BMQ / 32; ++mb) {
        __builtin_amdgcn_sched_barrier(0);
        f32x16 s = f32x16{}, dp = f32x16{};
        const T* qr = sQ + (32 * mb + l32) * C::P + 8 * h;
        const T* orr = sO + (32 * mb + l32) * C::P + 8 * h;
        // row reads kept RA k-steps ahead in a small ring (fenced, so that the
        // compiler does not hoist all KC of them into registers at once)
        constexpr int RA = 2;
        i32x4 aq[RA + 1], ao[RA + 1];
#pragma unroll
        for (int kc = 0; kc < RA; ++kc) {
          aq[kc] = lds_read16(qr + 16 * kc);
          if constexpr (DK) ao[kc] = lds_read16(orr + 16 * kc);
        }
#pragma unroll
        for (int kc = 0; kc < C::KC; ++kc) {
          __builtin_amdgcn_sched_barrier(0);
          if (kc + RA < C::KC) {
            aq[(kc + RA) % (RA + 1)] = lds_read16(qr + 16 * (kc + RA));
            if constexpr (DK) ao[(kc + RA) % (RA + 1)] = lds_read16(orr + 16 * (kc + RA));
          }
          s = M::mma(as_v8<V8>(aq[kc % (RA + 1)]), kf[kc], s);
          if constexpr (DK) dp = M::mma(as_v8<V8>(ao[kc % (RA + 1)]), vf[kc], dp);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int mr = 32 * mb + 8 * i + 4 * h;
          const f32x4 L = *(const f32x4*)&sL[mr];
          const f32x4 Dl = *(const f32x4*)&sDl[mr];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * i + j;
            const int m = mt + mr + j;
            float tv = 0.f;
            // m - my_n = (mt + 4h - my_n) + 32 mb + 8 i + j, exact in fp32
            const float y = score_log2_d<SOFTCAP, ALIBI>(s[r], p, slope_log2,
                                                         fq + (float)(32 * mb + 8 * i + j), tv);
            float pr = fast_exp2(y - L[j]);
            if (!full && (!allowed(p, m, my_n) || m < dlo || m >= dhi)) pr = 0.f;
            s[r] = pr;
            if constexpr (DK) {
              float ds = pr * (dp[r] - Dl[j]) * p.scale;
              if constexpr (SOFTCAP) ds *= (1.0f - tv * tv);
              dp[r] = ds;
            }
          }
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int row = 32 * mb + 16 * c + 4 * h + ((lane & 15) >> 2);
          const T* orow = sO + row * C::P + tr_col;
          const T* qrow = sQ + row * C::P + tr_col;
          // transpose reads one MFMA ahead (fenced: a two-entry ring)
          auto tr_mma = [&](const T* base, const V8 op, f32x16 (&acc)[C::DB]) {
            i16x4 lo[2], hi[2];
            lo[0] = lds_read_tr4(base);
            hi[0] = lds_read_tr4(base + 8 * C::P);
#pragma unroll
            for (int db = 0; db < C::DB; ++db) {
              __builtin_amdgcn_sched_barrier(0);
              if (db + 1 < C::DB) {
                lo[(db + 1) & 1] = lds_read_tr4(base + 32 * (db + 1));
                hi[(db + 1) & 1] = lds_read_tr4(base + 8 * C::P + 32 * (db + 1));
              }
              acc[db] = M::mma(cat_tr<V8>(lo[db & 1], hi[db & 1]), op, acc[db]);
            }
            __builtin_amdgcn_sched_barrier(0);
          };
          if constexpr (DV) tr_mma(orow, pack8<T>(s, 8 * c), adv);
          if constexpr (DK) tr_mma(qrow, pack8<T>(dp, 8 * c), adk);
        }
      }
    }
  };
  auto store = [&](const MutView& t, const f32x16 (&acc)[C::DB], float sc) {
    if (my_n < p.Skv) {
      T* dst = (T*)t.data + b * t.sb + hk * t.sh + (int64_t)my_n * t.ss + 4 * h;
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          st_global8(dst + 32 * db + 8 * i, pack4<T>(acc[db][4 * i] * sc, acc[db][4 * i + 1] * sc,
                                                    acc[db][4 * i + 2] * sc, acc[db][4 * i + 3] * sc));
    }
  };

  load_rows(a.k, kf);
  if constexpr (C::SPLIT) {
    // dV, then dK: only one accumulator set is live at a time
#pragma unroll
    for (int db = 0; db < C::DB; ++db) adv[db] = f32x16{};
    run(std::true_type{}, std::false_type{});
    store(a.dv, adv, 1.0f);
    load_rows(a.v, vf);
#pragma unroll
    for (int db = 0; db < C::DB; ++db) adk[db] = f32x16{};
    __syncthreads();  // the first pass's last tile has been read
    run(std::false_type{}, std::true_type{});
    store(a.dk, adk, 1.0f);
  } else {
    load_rows(a.v, vf);
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
      adk[db] = f32x16{};
      adv[db] = f32x16{};
    }
    run(std::true_type{}, std::true_type{});
    store(a.dv, adv, 1.0f);
    store(a.dk, adk, 1.0f);
  }
}

template <class T, int D>
hipError_t launch_dq_mfma(const BwdArgs& a, hipStream_t st) {
  using C = BwdCfg<D>;
  BwdArgs x = a;
  x.ntiles = (a.p.Sq + C::BM - 1) / C::BM;
  const dim3 grid(x.ntiles * a.p.B * a.p.Hq), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  if (sc && al) hipLaunchKernelGGL((bwd_dq_mfma_kernel<T, D, true, true>), grid, block, 0, st, x);
  else if (sc) hipLaunchKernelGGL((bwd_dq_mfma_kernel<T, D, true, false>), grid, block, 0, st, x);
  else if (al) hipLaunchKernelGGL((bwd_dq_mfma_kernel<T, D, false, true>), grid, block, 0, st, x);
  else hipLaunchKernelGGL((bwd_dq_mfma_kernel<T, D, false, false>), grid, block, 0, st, x);
  return hipGetLastError();
}

template <class T, int D>
hipError_t launch_dkdv_mfma(const BwdArgs& a, hipStream_t st) {
  using C = BwdCfg<D>;
  BwdArgs x = a;
  x.ntiles = (a.p.Skv + C::BNK - 1) / C::BNK;
  const dim3 grid(x.ntiles * a.p.B * a.p.Hkv), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  if (sc && al) hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, true, true>), grid, block, 0, st, x);
  else if (sc) hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, true, false>), grid, block, 0, st, x);
  else if (al) hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, false, true>), grid, block, 0, st, x);
  else hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, false, false>), grid, block, 0, st, x);
  return hipGetLastError();
}

#define FLEXATT_CAT2(a, b) a##b
#define FLEXATT_CAT(a, b) FLEXATT_CAT2(a, b)
hipError_t FLEXATT_CAT(bwd_dq_mfma_bf16_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  return launch_dq_mfma<__bf16, FLEXATT_D>(a, st);
}
hipError_t FLEXATT_CAT(bwd_dq_mfma_f16_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  return launch_dq_mfma<_Float16, FLEXATT_D>(a, st);
}
hipError_t FLEXATT_CAT(bwd_dkdv_mfma_bf16_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  return launch_dkdv_mfma<__bf16, FLEXATT_D>(a, st);
}
hipError_t FLEXATT_CAT(bwd_dkdv_mfma_f16_d, FLEXATT_D)(const BwdArgs& a, hipStream_t st) {
  return launch_dkdv_mfma<_Float16, FLEXATT_D>(a, st);
}

}  // namespace flexatt

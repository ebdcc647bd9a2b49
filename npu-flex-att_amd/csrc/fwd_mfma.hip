// Flash-attention forward for fp16/bf16 on gfx950 MFMA.
//
// Semantics: npu_flash_attention.py:17-166 (flash_attn_fwd_kernel) — online
// softmax over KV tiles, O in the input dtype, LSE in fp32 natural log, the
// score order scale -> soft-cap -> ALiBi -> mask, GQA head h -> h / G.
//
// Decomposition (one workgroup = 4 waves = 128 query rows of one (b, hq)):
//  * each wave owns 32 query rows and computes S^T = K Q^T per 32x32 block
//    (A = K rows from LDS, B = its Q rows held in registers), so every lane
//    holds one query row: the row max needs one exchange between the two wave
//    halves and the O rescale is a per-lane scalar;
//  * O^T = V^T P^T, with P^T taken straight from the S^T accumulators and V^T
//    read from the row-major V tile with the LDS transpose read;
//  * K/V tiles of 64 rows are staged in LDS; the next tile's global loads are
//    issued into registers before the current tile is computed;
//  * causal/window tiles outside a wave's rows are skipped; only tiles that
//    straddle a mask edge or the KV tail evaluate the mask per element.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

template <int D>
struct FwdCfg {
  static constexpr int NW = 4;
  static constexpr int BM = 32 * NW;
  static constexpr int BN = 64;
  static constexpr int KC = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int P = D + 8;  // LDS row pitch (elements)
  static constexpr int CPR = D / 8;  // 16-byte chunks per row
  static constexpr int CPT = BN * CPR / (NW * 64);  // chunks per thread per tile
  static constexpr bool PREFETCH = D <= 128;
};

template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(256) void fwd_mfma_kernel(FwdArgs a) {
  using C = FwdCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(16))) T sK[C::BN * C::P];
  __shared__ __attribute__((aligned(16))) T sV[C::BN * C::P];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;

  // (b, hq, q-tile); the longest causal tiles are dispatched first.
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = a.nqt - 1 - (w % a.nqt);
  const int bh = w / a.nqt;
  const int hq = bh % p.Hq, b = bh / p.Hq;
  const int hk = hq / p.G;
  const int m0 = qt * C::BM;
  const int mw = m0 + wave * 32;
  const int my_m = mw + l32;

  const T* qp = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh;
  const T* kp = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const T* vp = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh;

  V8 qf[C::KC];
  {
    const int r = min(my_m, p.Sq - 1);
    const T* src = qp + (int64_t)r * a.q.ss + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      i32x4 x = ld_global16(src + 16 * kc);
      if (my_m >= p.Sq) x = i32x4{0, 0, 0, 0};
      qf[kc] = as_v8<V8>(x);
    }
  }

  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + C::BM);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
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
      i32x4 xk = ld_global16(kp + (int64_t)nc * a.k.ss + col);
      i32x4 xv = ld_global16(vp + (int64_t)nc * a.v.ss + col);
      if (n >= p.Skv) { xk = i32x4{0, 0, 0, 0}; xv = i32x4{0, 0, 0, 0}; }
      rk[e] = xk;
      rv[e] = xv;
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
  float m_run = kNegInf, l_run = 0.f;
  const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;

  if (C::PREFETCH && t_lo < t_hi) gload(t_lo);
  for (int t = t_lo; t < t_hi; ++t) {
    if (t > t_lo) __syncthreads();
    if (!C::PREFETCH) gload(t);
    lstore();
    __syncthreads();
    if (C::PREFETCH && t + 1 < t_hi) gload(t + 1);

    const int n0 = t * C::BN;
    const bool skip = (p.causal && n0 > mw + 31) || (p.window > 0 && mw - (n0 + C::BN - 1) > p.window);
    if (skip) continue;
    const bool full = (n0 + C::BN <= p.Skv) && (!p.causal || n0 + C::BN - 1 <= mw) &&
                      (p.window == 0 || mw + 31 - n0 <= p.window);

    f32x16 s[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      s[bb] = f32x16{};
      const T* kr = sK + (32 * bb + l32) * C::P + 8 * h;
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc) s[bb] = M::mma(as_v8<V8>(lds_read16(kr + 16 * kc)), qf[kc], s[bb]);
    }

    float mx = kNegInf;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = n0 + 32 * bb + 8 * (r >> 2) + 4 * h + (r & 3);
        float tv;
        float y = score_log2<SOFTCAP, ALIBI>(s[bb][r], p, slope_log2, my_m, j, tv);
        if (!full && !allowed(p, my_m, j)) y = kNegInf;
        s[bb][r] = y;
        mx = fmaxf(mx, y);
      }
    }
    mx = fmaxf(mx, swap_halves(mx));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float rs = 0.f;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(s[bb][r] - m_use);
        s[bb][r] = e;
        rs += e;
      }
    }
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < C::DB; ++db) acc[db] *= alpha;

    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const V8 pb = pack8<T>(s[bb], 8 * c);
        const int row = 32 * bb + 16 * c + 4 * h + ((lane & 15) >> 2);
        const T* vr = sV + row * C::P + tr_col;
#pragma unroll
        for (int db = 0; db < C::DB; ++db) {
          const i16x4 lo = lds_read_tr4(vr + 32 * db);
          const i16x4 hi = lds_read_tr4(vr + 8 * C::P + 32 * db);
          acc[db] = M::mma(cat_tr<V8>(lo, hi), pb, acc[db]);
        }
      }
    }
  }

  const float l_tot = l_run + swap_halves(l_run);
  const bool empty = !(l_tot > 0.f);
  const float inv = empty ? 0.f : 1.0f / l_tot;
  if (my_m < p.Sq) {
    T* op = (T*)a.o.data + b * a.o.sb + hq * a.o.sh + (int64_t)my_m * a.o.ss + 4 * h;
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st_global8(op + 32 * db + 8 * i,
                   pack4<T>(acc[db][4 * i] * inv, acc[db][4 * i + 1] * inv, acc[db][4 * i + 2] * inv,
                            acc[db][4 * i + 3] * inv));
      }
    }
    if (h == 0) a.lse[(int64_t)(b * p.Hq + hq) * p.Sq + my_m] = empty ? kNegInf : (m_run + log2f(l_tot)) * kLn2;
  }
}

template <class T, int D>
hipError_t launch_fwd_mfma(const FwdArgs& a, hipStream_t st) {
  using C = FwdCfg<D>;
  FwdArgs x = a;
  x.nqt = (a.p.Sq + C::BM - 1) / C::BM;
  const dim3 grid(x.nqt * a.p.B * a.p.Hq), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  if (sc && al) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, true, true>), grid, block, 0, st, x);
  else if (sc) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, true, false>), grid, block, 0, st, x);
  else if (al) hipLaunchKernelGGL((fwd_mfma_kernel<T, D, false, true>), grid, block, 0, st, x);
  else hipLaunchKernelGGL((fwd_mfma_kernel<T, D, false, false>), grid, block, 0, st, x);
  return hipGetLastError();
}

#define FLEXATT_CAT2(a, b) a##b
#define FLEXATT_CAT(a, b) FLEXATT_CAT2(a, b)
hipError_t FLEXATT_CAT(fwd_mfma_bf16_d, FLEXATT_D)(const FwdArgs& a, hipStream_t st) {
  return launch_fwd_mfma<__bf16, FLEXATT_D>(a, st);
}
hipError_t FLEXATT_CAT(fwd_mfma_f16_d, FLEXATT_D)(const FwdArgs& a, hipStream_t st) {
  return launch_fwd_mfma<_Float16, FLEXATT_D>(a, st);
}

}  // namespace flexatt

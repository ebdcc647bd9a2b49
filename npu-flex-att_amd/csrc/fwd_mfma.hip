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
//  * K/V tiles of 64 rows are double-buffered in LDS (one barrier per tile);
//    the next tile's global loads are issued into registers before the current
//    tile is computed.  Row pitches: K = D+8 elements (conflict-free 16-byte
//    column reads), V = D+16 (conflict-free transpose reads);
//  * two workgroups per CU (<= 256 registers per lane) so that one wave's
//    softmax overlaps the other's MFMAs;
//  * lazy rescale: the running max only moves when a row's max grows by more
//    than 2^8, so O is rescaled rarely; P <= 2^8 stays exact in fp16/bf16 and
//    the final O / l and LSE use the same max, so results are unchanged;
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
  static constexpr int KP = D + 8;   // K tile pitch (elements)
  static constexpr int VP = D + 16;  // V tile pitch (elements)
  static constexpr int CPR = D / 8;  // 16-byte chunks per row
  static constexpr int CPT = BN * CPR / (NW * 64);  // chunks per thread per tile
  static constexpr int NBUF = D <= 128 ? 2 : 1;
  static constexpr int SK = BN * KP, SV = BN * VP;
  static constexpr int WPE = D <= 128 ? 2 : 1;  // waves per SIMD the register budget targets
};

constexpr float kRescaleThreshold = 8.0f;  // log2 units

template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(FwdCfg<D>::WPE, FwdCfg<D>::WPE)))
void fwd_mfma_kernel(FwdArgs a) {
  using C = FwdCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(16))) T smem[C::NBUF * (C::SK + C::SV)];

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

  // Next-tile staging: K(t+1) is loaded at the start of tile t and written to
  // the free LDS buffer after the first 32-row block; V(t+1) is loaded then
  // and written at the end of the tile.  Half a tile of registers is live.
  i32x4 rs[C::CPT];
  auto gload = [&](const T* base, int64_t ss, int t) {
    const int n0 = t * C::BN;
#pragma unroll
    for (int e = 0; e < C::CPT; ++e) {
      const int c = tid + e * C::NW * 64;
      const int row = c / C::CPR, col = (c % C::CPR) * 8;
      const int n = n0 + row;
      i32x4 x = ld_global16(base + (int64_t)min(n, p.Skv - 1) * ss + col);
      if (n >= p.Skv) x = i32x4{0, 0, 0, 0};
      rs[e] = x;
    }
  };
  auto lstore = [&](T* dst, int pitch) {
#pragma unroll
    for (int e = 0; e < C::CPT; ++e) {
      const int c = tid + e * C::NW * 64;
      const int row = c / C::CPR, col = (c % C::CPR) * 8;
      *(i32x4*)&dst[row * pitch + col] = rs[e];
    }
  };

  f32x16 acc[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) acc[db] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;
  const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;
  const float c2 = p.scale_log2;
  const int tr_row = 4 * h + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // One 32-row KV block: S^T, online-softmax update, O^T += V^T P^T.
  auto block = [&](int n0, const T* sK, const T* sV, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    f32x16 s = f32x16{};
    const T* kr = sK + l32 * C::KP + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) s = M::mma(as_v8<V8>(lds_read16(kr + 16 * kc)), qf[kc], s);

    // log2-domain scores; the fast path keeps raw scores and folds the scale
    // into the exponent's FMA.
    constexpr bool RAW = !SOFTCAP && !ALIBI && !MASK;
    float mx = kNegInf;
    if constexpr (RAW) {
      float hi = kNegInf, lo = __builtin_huge_valf();
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        hi = fmaxf(hi, s[r]);
        lo = fminf(lo, s[r]);
      }
      mx = c2 >= 0.f ? hi * c2 : lo * c2;
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = n0 + 8 * (r >> 2) + 4 * h + (r & 3);
        float tv;
        float y = score_log2<SOFTCAP, ALIBI>(s[r], p, slope_log2, my_m, j, tv);
        if constexpr (MASK) {
          if (!allowed(p, my_m, j)) y = kNegInf;
        }
        s[r] = y;
        mx = fmaxf(mx, y);
      }
    }
    mx = fmaxf(mx, swap_halves(mx));
    const bool grow = mx > m_run + kRescaleThreshold;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) acc[db] *= alpha;
      m_run = m_new;
    }
    const float m_use = (m_run == kNegInf) ? 0.f : m_run;
    float rsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float e;
      if constexpr (RAW) e = fast_exp2(__builtin_fmaf(s[r], c2, -m_use));
      else e = fast_exp2(s[r] - m_use);
      s[r] = e;
      rsum += e;
    }
    l_run += rsum;

#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const V8 pb = pack8<T>(s, 8 * c);
      const T* vr = sV + (16 * c + tr_row) * C::VP + tr_col;
#pragma unroll
      for (int db = 0; db < C::DB; ++db) {
        const i16x4 lo = lds_read_tr4(vr + 32 * db);
        const i16x4 hi = lds_read_tr4(vr + 8 * C::VP + 32 * db);
        acc[db] = M::mma(cat_tr<V8>(lo, hi), pb, acc[db]);
      }
    }
  };

  if (t_lo < t_hi) {
    gload(kp, a.k.ss, t_lo);
    lstore(smem, C::KP);
    gload(vp, a.v.ss, t_lo);
    lstore(smem + C::SK, C::VP);
  }
  __syncthreads();
  for (int t = t_lo; t < t_hi; ++t) {
    const int cur = C::NBUF == 2 ? ((t - t_lo) & 1) : 0;
    const bool more = t + 1 < t_hi;
    T* sK = smem + cur * (C::SK + C::SV);
    T* sV = sK + C::SK;
    T* nK = smem + (cur ^ 1) * (C::SK + C::SV);
    T* nV = nK + C::SK;
    const int n0 = t * C::BN;
    if constexpr (C::NBUF == 2) {
      if (more) gload(kp, a.k.ss, t + 1);
    }
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const int nb = n0 + 32 * bb;
      const bool skip = (p.causal && nb > mw + 31) || (p.window > 0 && mw - (nb + 31) > p.window);
      if (!skip) {
        const bool full = (nb + 32 <= p.Skv) && (!p.causal || nb + 31 <= mw) &&
                          (p.window == 0 || mw + 31 - nb <= p.window);
        if (full) block(nb, sK + 32 * bb * C::KP, sV + 32 * bb * C::VP, std::false_type{});
        else block(nb, sK + 32 * bb * C::KP, sV + 32 * bb * C::VP, std::true_type{});
      }
      if constexpr (C::NBUF == 2) {
        if (bb == 0 && more) {
          lstore(nK, C::KP);
          gload(vp, a.v.ss, t + 1);
        }
      }
    }
    if constexpr (C::NBUF == 2) {
      if (more) lstore(nV, C::VP);
      __syncthreads();
    } else {
      __syncthreads();
      if (more) {
        gload(kp, a.k.ss, t + 1);
        lstore(sK, C::KP);
        gload(vp, a.v.ss, t + 1);
        lstore(sV, C::VP);
      }
      __syncthreads();
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

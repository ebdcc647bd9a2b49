// Flash-attention backward dK/dV for fp16/bf16 on gfx950 MFMA (KV-stationary
// tile stream).
//
// Semantics: npu_flash_attention.py:407-560 (flash_attn_bwd_dkdv_kernel) plus
// the group sum at :734-737: P is recomputed from the forward LSE (including
// the ALiBi bias, which the reference's backward kernels omit),
// dP = dO V^T, dS = P (dP - Delta) scale (1 - tanh^2), dV = sum_h P^T dO,
// dK = sum_h dS^T Q over the G query heads h of a KV head, accumulated in
// fp32 and written once as [B, Hkv, Skv, D].  P and dS are rounded to the
// input dtype before their MFMAs, as the reference does before tl.dot.
//
// Decomposition
//  * One workgroup = 4 waves (one per SIMD, the whole register file each) =
//    128 KV rows of one (b, hkv); each wave owns 32 KV rows and each lane one
//    KV row: its K and V rows stay in registers as MFMA B operands and its
//    dK^T / dV^T columns accumulate in registers.
//  * The workgroup walks one stream of tiles: for each of the G query heads of
//    the group, the 32-row query tiles that can attend to its KV rows.  A tile
//    is Q, dO (32 x D each), LSE and Delta (32 floats each), copied global ->
//    LDS with direct-to-LDS loads two tiles ahead into four stages (one
//    barrier per tile, no staging registers).
//  * Q and dO are read two ways from the same tile, as rows (S = Q K^T,
//    dP = dO V^T) and as columns (dV^T += dO^T P, dK^T += Q^T dS, with the LDS
//    transpose read); the dual-use swizzle keeps both conflict-free.
//  * Software pipeline inside each wave: the S / dP MFMAs of tile u are issued
//    first; then the dV / dK MFMAs of tile u-1 run while the VALU forms P and
//    dS of tile u.
//  * Tiles that cross the causal diagonal, the window edge or the Q / KV
//    tails take the fast path first and then recompute P and dS with the
//    per-element mask (only the packed P / dS registers differ between the two
//    paths, so the accumulators never sit on two code paths).
// Deterministic: every output element is owned by one lane and accumulated in
// a fixed order.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

#if FLEXATT_D == 128

template <int D>
struct KvCfg {
  static constexpr int NW = 4;          // waves per workgroup, one per SIMD
  static constexpr int BKV = 32 * NW;   // KV rows per workgroup
  static constexpr int BM = 32;         // query rows per tile
  static constexpr int QB = BM / 32;
  static constexpr int KC = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CPR = D / 8;
  static constexpr int ROWB = 2 * D;
  static constexpr int TILEB = BM * ROWB;              // one of Q / dO
  static constexpr int E = TILEB / (1024 * NW);        // 1 KB copies per wave per tensor
  static constexpr int STAGEB = 2 * TILEB + 2 * BM * 4;  // Q, dO, LSE, Delta
  static constexpr int STAGES = 4;
  static constexpr int NPK = 2 * QB;                   // packed P (or dS) operands per tile
  static_assert(E * 1024 * NW == TILEB, "tile must split into 1 KB copies");
  static constexpr int RPW = BM / NW;                  // LSE / Delta values copied per wave
  static_assert(RPW * NW == BM && RPW <= 64, "LSE / Delta rows split over the waves");
};

template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void bwd_kv_kernel(BwdArgs a) {
  using C = KvCfg<D>;
  static_assert(C::QB == 1 && C::DB == 4, "the hand-ordered step assumes one 32-row query block and D = 128");
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(1024))) char smem[C::STAGES * C::STAGEB];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;

  // Work item: (b, hkv, KV block), blocks of one (b, hkv) consecutive so that
  // they share an XCD (and its L2) and heavy / light causal blocks interleave.
  const int nkb = a.ntiles;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int kb = w % nkb, bh = w / nkb;
  const int hk = bh % p.Hkv, b = bh / p.Hkv;
  const int n0 = kb * C::BKV;
  const int kw0 = n0 + 32 * wave;  // first KV row of this wave
  const int my_kv = kw0 + l32;     // KV row of this lane

  // Query rows that can attend to this block's KV rows.  (64-row query tiles
  // at 128 KV rows per workgroup would need more than the 256 VGPRs a wave can
  // address for scores, dP and two sets of packed P / dS.)
  int q_lo = 0, q_hi = p.Sq;
  if (p.causal) q_lo = n0;  // q >= kv >= n0
  if (p.window > 0) q_hi = min(q_hi, n0 + C::BKV + p.window);  // q - kv <= W
  const int qt_lo = q_lo / C::BM;
  const int nqt = q_hi > q_lo ? (q_hi + C::BM - 1) / C::BM - qt_lo : 0;
  const int ntile = p.G * nqt;

  // K / V rows as MFMA B operands (lane = KV row, k = 8 consecutive d).
  V8 kreg[C::KC], vreg[C::KC];
  {
    const int r = min(my_kv, p.Skv - 1);
    const T* kr = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh + (int64_t)r * a.k.ss + 8 * h;
    const T* vr = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh + (int64_t)r * a.v.ss + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      kreg[kc] = as_v8<V8>(ld_global16(kr + 16 * kc));
      vreg[kc] = as_v8<V8>(ld_global16(vr + 16 * kc));
    }
  }
  f32x16 dk[C::DB], dv[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }

  // Tile copies: tile u -> stage u % 4; past the end, redundant copies of the
  // last tile into a free stage keep every wave at 2E + 2 operations per tile.
  const unsigned lds0 = lds_addr_of(smem);
  int crow[C::E], cchk[C::E];  // row / logical chunk of this lane in copy e
#pragma unroll
  for (int e = 0; e < C::E; ++e) {
    const int q = (wave * C::E + e) * 64 + lane;
    crow[e] = q / C::CPR;
    cchk[e] = swz_dual_inv<C::CPR>(crow[e], q % C::CPR);
  }
  int is_g = 0, is_qt = qt_lo;  // next tile to copy (head, query tile)
  auto issue = [&](int u) {
    const unsigned sb = lds0 + (u & 3) * C::STAGEB;
    const int hq = hk * p.G + min(is_g, p.G - 1);
    const int m0 = (is_g < p.G ? is_qt : qt_lo + nqt - 1) * C::BM;
    const T* qg = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh;
    const T* og = (const T*)a.dout.data + b * a.dout.sb + hq * a.dout.sh;
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int64_t r = min(m0 + crow[e], p.Sq - 1);
      const unsigned dst = sb + (wave * C::E + e) * 1024;
      load_lds16(qg + r * a.q.ss + cchk[e] * 8, dst);
      load_lds16(og + r * a.dout.ss + cchk[e] * 8, dst + C::TILEB);
    }
    const int64_t rr = (int64_t)(b * p.Hq + hq) * p.Sq + min(m0 + C::RPW * wave + lane, p.Sq - 1);
    if (lane < C::RPW) {
      load_lds4(a.lse + rr, sb + 2 * C::TILEB + 4 * C::RPW * wave);
      load_lds4(a.delta + rr, sb + 2 * C::TILEB + C::BM * 4 + 4 * C::RPW * wave);
    }
    if (++is_qt == qt_lo + nqt) {
      is_qt = qt_lo;
      ++is_g;
    }
  };
  auto wait_tile = [&]() { wait_vmcnt<2 * C::E + 2>(); };

  // Lane-constant LDS byte offsets.
  int koff[C::KC], voff_lo[C::DB], voff_hi[C::DB];
#pragma unroll
  for (int kc = 0; kc < C::KC; ++kc) koff[kc] = l32 * C::ROWB + swz_dual<C::CPR>(l32, 2 * kc + h) * 16;
  {
    const int tr_row = 4 * h + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
      const int c = 4 * db + (tr_col >> 3), e2 = (tr_col & 7) * 2;
      voff_lo[db] = tr_row * C::ROWB + swz_dual<C::CPR>(tr_row, c) * 16 + e2;
      voff_hi[db] = (tr_row + 8) * C::ROWB + swz_dual<C::CPR>(tr_row + 8, c) * 16 + e2;
    }
  }

  constexpr bool RAW = !SOFTCAP && !ALIBI;
  const float c2 = p.scale_log2;

  f32x16 S[C::QB], DP[C::QB];  // scores and dP of the tile being processed
  V8 PP[C::NPK], PS[C::NPK];    // packed P and dS of the previous tile

  // S = Q K^T and dP = dO V^T of the tile in stage st (lane = KV row).
  auto mma_s = [&](int st) {
    const char* sQ = smem + st * C::STAGEB;
    const char* sO = sQ + C::TILEB;
#pragma unroll
    for (int qb = 0; qb < C::QB; ++qb) {
      S[qb] = f32x16{};
      DP[qb] = f32x16{};
    }
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
#pragma unroll
      for (int qb = 0; qb < C::QB; ++qb)
        S[qb] = M::mma(as_v8<V8>(lds_read16(sQ + qb * 32 * C::ROWB + koff[kc])), kreg[kc], S[qb]);
#pragma unroll
      for (int qb = 0; qb < C::QB; ++qb)
        DP[qb] = M::mma(as_v8<V8>(lds_read16(sO + qb * 32 * C::ROWB + koff[kc])), vreg[kc], DP[qb]);
    }
  };

  // dV^T += dO^T P and dK^T += Q^T dS for the tile in stage st.
  auto mma_kv = [&](int st) {
    const char* sQ = smem + st * C::STAGEB;
    const char* sO = sQ + C::TILEB;
#pragma unroll
    for (int qb = 0; qb < C::QB; ++qb)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int rb = (32 * qb + 16 * c) * C::ROWB;
#pragma unroll
        for (int db = 0; db < C::DB; ++db) {
          const i16x4 olo = lds_read_tr4(sO + rb + voff_lo[db]);
          const i16x4 ohi = lds_read_tr4(sO + rb + voff_hi[db]);
          dv[db] = M::mma(cat_tr<V8>(olo, ohi), PP[2 * qb + c], dv[db]);
          const i16x4 qlo = lds_read_tr4(sQ + rb + voff_lo[db]);
          const i16x4 qhi = lds_read_tr4(sQ + rb + voff_hi[db]);
          dk[db] = M::mma(cat_tr<V8>(qlo, qhi), PS[2 * qb + c], dk[db]);
        }
      }
  };

  // LSE and Delta of this lane's 4 * QB * 4 query rows of the tile in stage st.
  f32x4 L4[C::QB * 4], D4[C::QB * 4];
  auto read_rows = [&](int st) {
    const float* sL = (const float*)(smem + st * C::STAGEB + 2 * C::TILEB);
    const float* sD = sL + C::BM;
#pragma unroll
    for (int qb = 0; qb < C::QB; ++qb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ro = 32 * qb + 8 * i + 4 * h;
        L4[4 * qb + i] = __builtin_bit_cast(f32x4, lds_read16(sL + ro));
        D4[4 * qb + i] = __builtin_bit_cast(f32x4, lds_read16(sD + ro));
      }
  };

  // P and dS of the current tile (query rows m0.., LSE / Delta in L4 / D4)
  // from S / DP.  MASKED: per-element mask, query tail, and exact zeros for
  // masked pairs.
  auto valu = [&](int m0, float slope_log2, bool masked, V8 (&pp)[C::NPK], V8 (&ps)[C::NPK]) {
#pragma unroll
    for (int qb = 0; qb < C::QB; ++qb) {
      f32x16 pe, de;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ro = 32 * qb + 8 * i + 4 * h;
        const f32x4 l4 = L4[4 * qb + i];
        const f32x4 d4 = D4[4 * qb + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * i + j;
          const int q = m0 + ro + j;
          const float l2 = l4[j] * kLog2e;
          float e, t = 0.f;
          if constexpr (RAW) {
            e = fast_exp2(__builtin_fmaf(S[qb][r], c2, -l2));
          } else {
            const float y = score_log2<SOFTCAP, ALIBI>(S[qb][r], p, slope_log2, q, my_kv, t);
            e = fast_exp2(y - l2);
          }
          if (masked) {
            // branch-free: every term evaluated, one select
            const bool ok = (q < p.Sq) & (my_kv < p.Skv) & (!p.causal | (my_kv <= q)) &
                            ((p.window == 0) | (q - my_kv <= p.window));
            e = ok ? e : 0.f;
          }
          float ds = e * (DP[qb][r] - d4[j]);
          if constexpr (SOFTCAP) ds *= 1.f - t * t;
          pe[r] = e;
          de[r] = ds;
        }
      }
      pp[2 * qb] = pack8<T>(pe, 0);
      pp[2 * qb + 1] = pack8<T>(pe, 8);
      ps[2 * qb] = pack8<T>(de, 0);
      ps[2 * qb + 1] = pack8<T>(de, 8);
    }
  };

  // Which tiles need the per-element pass, for this wave's KV rows
  // [kw0, kw0 + 32): query tail, KV tail, causal diagonal, window edge.
  auto need_mask = [&](int m0) {
    return (m0 + C::BM > p.Sq) || (kw0 + 32 > p.Skv) || (p.causal && m0 < kw0 + 31) ||
           (p.window > 0 && m0 + C::BM - 1 - kw0 > p.window);
  };

  int cg = 0, cqt = qt_lo;  // tile being computed (head, query tile)
  auto tile_info = [&](int& m0, float& slope) {
    const int hq = hk * p.G + cg;
    m0 = cqt * C::BM;
    slope = ALIBI ? p.alibi[hq] * kLog2e : 0.f;
    if (++cqt == qt_lo + nqt) {
      cqt = qt_lo;
      ++cg;
    }
  };

  if (ntile > 0) {
    issue(0);
    issue(1);
    // u = 0: S / dP and P / dS only
    {
      wait_tile();
      __syncthreads();
      issue(2);
      int m0;
      float sl;
      tile_info(m0, sl);
      mma_s(0);
      read_rows(0);
      valu(m0, sl, false, PP, PS);
      if (need_mask(m0)) valu(m0, sl, true, PP, PS);
    }
    for (int u = 1; u < ntile; ++u) {
      wait_tile();
      __syncthreads();  // tile u landed; stage (u - 2) % 4 no longer read
      issue(u + 2);
      int m0;
      float sl;
      tile_info(m0, sl);
      const int st = u & 3, sp = (u - 1) & 3;
      // Region A: S / dP MFMAs, row reads four steps ahead, then this tile's
      // LSE / Delta rows.  Each step is fenced so the order is kept as written.
      {
        const char* sQ = smem + st * C::STAGEB;
        const char* sO = sQ + C::TILEB;
        constexpr int NA = 2 * C::KC;
        auto rdA = [&](int k) { return lds_read16((k & 1 ? sO : sQ) + koff[k >> 1]); };
        i32x4 ab[5];
#pragma unroll
        for (int k = 0; k < 4; ++k) ab[k] = rdA(k);
        S[0] = f32x16{};
        DP[0] = f32x16{};
#pragma unroll
        for (int k = 0; k < NA; ++k) {
          __builtin_amdgcn_sched_barrier(0);
          if (k + 4 < NA) ab[(k + 4) % 5] = rdA(k + 4);
          if (k & 1) DP[0] = M::mma(as_v8<V8>(ab[k % 5]), vreg[k >> 1], DP[0]);
          else S[0] = M::mma(as_v8<V8>(ab[k % 5]), kreg[k >> 1], S[0]);
          if (k == NA - 4) read_rows(st);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // Region B: dV / dK MFMAs of the previous tile, transpose reads two
      // steps ahead; after MFMA k, element k of this tile's P and dS.
      V8 PPn[C::NPK], PSn[C::NPK];
      {
        const char* sQp = smem + sp * C::STAGEB;
        const char* sOp = sQp + C::TILEB;
        constexpr int NB = 4 * C::QB * C::DB;
        auto rdB = [&](int k, i16x4& lo, i16x4& hi) {
          const int db = (k >> 1) % C::DB, qc = (k >> 1) / C::DB;
          const char* base = ((k & 1) ? sQp : sOp) + 16 * qc * C::ROWB;
          lo = lds_read_tr4(base + voff_lo[db]);
          hi = lds_read_tr4(base + voff_hi[db]);
        };
        i16x4 blo[3], bhi[3];
        rdB(0, blo[0], bhi[0]);
        rdB(1, blo[1], bhi[1]);
        f32x16 pe, de;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
          __builtin_amdgcn_sched_barrier(0);
          if (k + 2 < NB) rdB(k + 2, blo[(k + 2) % 3], bhi[(k + 2) % 3]);
          const int db = (k >> 1) % C::DB, qc = (k >> 1) / C::DB;
          if (k & 1) dk[db] = M::mma(cat_tr<V8>(blo[k % 3], bhi[k % 3]), PS[qc], dk[db]);
          else dv[db] = M::mma(cat_tr<V8>(blo[k % 3], bhi[k % 3]), PP[qc], dv[db]);
          // element r = k of the current tile (one 32-row query block)
          const int r = k, i = r >> 2, j = r & 3;
          const int q = m0 + 8 * i + 4 * h + j;
          const float l2 = L4[i][j] * kLog2e;
          float e, t = 0.f;
          if constexpr (RAW) {
            e = fast_exp2(__builtin_fmaf(S[0][r], c2, -l2));
          } else {
            const float y = score_log2<SOFTCAP, ALIBI>(S[0][r], p, sl, q, my_kv, t);
            e = fast_exp2(y - l2);
          }
          float ds = e * (DP[0][r] - D4[i][j]);
          if constexpr (SOFTCAP) ds *= 1.f - t * t;
          pe[r] = e;
          de[r] = ds;
          if (r == 7) {
            PPn[0] = pack8<T>(pe, 0);
            PSn[0] = pack8<T>(de, 0);
          } else if (r == 15) {
            PPn[1] = pack8<T>(pe, 8);
            PSn[1] = pack8<T>(de, 8);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // fast-path P / dS stay computed here (not sunk into the branch below)
#pragma unroll
      for (int i = 0; i < C::NPK; ++i) {
        pin(PPn[i]);
        pin(PSn[i]);
      }
      if (need_mask(m0)) valu(m0, sl, true, PPn, PSn);
#pragma unroll
      for (int i = 0; i < C::NPK; ++i) {
        PP[i] = PPn[i];
        PS[i] = PSn[i];
      }
    }
    mma_kv((ntile - 1) & 3);
    wait_vmcnt<0>();  // redundant copies in flight must land before the workgroup ends
  }

  // dK = scale * sum dS^T Q, dV = sum P^T dO; lane = KV row.
  if (my_kv < p.Skv) {
    T* kq = (T*)a.dk.data + b * a.dk.sb + hk * a.dk.sh + (int64_t)my_kv * a.dk.ss + 4 * h;
    T* vq = (T*)a.dv.data + b * a.dv.sb + hk * a.dv.sh + (int64_t)my_kv * a.dv.ss + 4 * h;
    const float sc = p.scale;
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st_global8(kq + 32 * db + 8 * i, pack4<T>(dk[db][4 * i] * sc, dk[db][4 * i + 1] * sc,
                                                 dk[db][4 * i + 2] * sc, dk[db][4 * i + 3] * sc));
        st_global8(vq + 32 * db + 8 * i, pack4<T>(dv[db][4 * i], dv[db][4 * i + 1], dv[db][4 * i + 2],
                                                 dv[db][4 * i + 3]));
      }
  }
}

template <class T, int D>
hipError_t launch_kv(const BwdArgs& a, hipStream_t st) {
  using C = KvCfg<D>;
  BwdArgs x = a;
  x.ntiles = (a.p.Skv + C::BKV - 1) / C::BKV;
  const dim3 grid(x.ntiles * a.p.B * a.p.Hkv), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  if (sc && al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, true>), grid, block, 0, st, x);
  else if (sc) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, false>), grid, block, 0, st, x);
  else if (al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, true>), grid, block, 0, st, x);
  else hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, false>), grid, block, 0, st, x);
  return hipGetLastError();
}

hipError_t bwd_kv_bf16_d128(const BwdArgs& a, hipStream_t st) { return launch_kv<__bf16, 128>(a, st); }
hipError_t bwd_kv_f16_d128(const BwdArgs& a, hipStream_t st) { return launch_kv<_Float16, 128>(a, st); }

#endif  // FLEXATT_D == 128

}  // namespace flexatt

// Flash-attention backward dQ for fp16/bf16 on gfx950 MFMA (query-stationary
// tile stream, KV-split wave pairs).
//
// Semantics: npu_flash_attention.py:298-402 (flash_attn_bwd_dq_kernel): P is
// recomputed from the forward LSE (including the ALiBi bias, which the
// reference's backward kernels omit), dP = dO V^T,
// dS = P (dP - Delta) scale (1 - tanh^2), dQ = dS K; dS is rounded to the
// input dtype before its MFMA, as the reference does before tl.dot.
//
// Decomposition
//  * One workgroup = 8 waves for one (batch, KV head): gp query heads that
//    share it (gp = the largest power of two dividing G, at most 4) and
//    32 * 4 / gp query rows of each.  Query slot s (32 rows of one head) is
//    owned by the wave pair s, s + 4, which share a SIMD: lane = query row, the
//    Q and dO rows in registers as MFMA B operands in both waves.  Each 64-row
//    KV tile is split between the pair: wave s takes KV rows 0-31, wave s + 4
//    rows 32-63.  Each wave accumulates its own partial dQ^T; the two partials
//    are added once, through LDS, at the end (fixed order: deterministic).
//  * Per tile and wave: S^T = K Q^T and dP^T = V dO^T for its 32 KV rows (A =
//    K / V rows from LDS, 16 MFMAs), P and dS on the VALU, then
//    dQ^T += K^T dS^T (8 MFMAs, K^T read with the LDS transpose read from the
//    same swizzled K tile).
//  * Ping-pong: the two halves run the same program one phase apart.  An MFMA
//    phase issues the S / dP MFMAs of tile t and the dQ MFMAs of tile t-1
//    (24 independent MFMAs); a VALU phase forms P and dS of tile t.  While
//    one wave of a SIMD streams MFMAs the other runs its VALU phase.
//  * K / V tiles are copied global -> LDS with direct-to-LDS loads two tiles
//    ahead into four stages, issued in the VALU phases; every phase ends with
//    a workgroup barrier.
//  * Fused Delta (a.delta_out set): each wave also loads its O rows with the
//    Q / dO rows and forms Delta = sum_d O dO of its rows itself (fp32, a
//    fixed order); the first wave of each pair writes it for the dK/dV
//    kernel, so the separate Delta pass (npu_flash_attention.py:681-685) is
//    not launched.
// Deterministic: every output element is owned by one lane pair and
// accumulated in a fixed order.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

#if FLEXATT_D == 128 || FLEXATT_D == 64

template <int D>
struct QCfg {
  static constexpr int NS = 4;        // query slots per workgroup (one per SIMD)
  static constexpr int NW = 2 * NS;   // waves: slot s and s + 4 split each KV tile
  static constexpr int BN = 64;       // KV rows per tile (32 per wave)
  static constexpr int KC = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CPR = D / 8;
  static constexpr int ROWB = 2 * D;
  static constexpr int TILEB = BN * ROWB;         // one of K / V
  static constexpr int E = TILEB / (1024 * NW);   // 1 KB copies per wave per tensor
  static constexpr int STAGEB = 2 * TILEB;
  static constexpr int STAGES = 4;
  static constexpr int RA = 4;  // row reads issued this many MFMAs ahead
  static constexpr int RB = 3;  // transpose reads issued this many dQ MFMAs ahead
  static_assert(E * 1024 * NW == TILEB, "tile must split into 1 KB copies");
  static_assert(4 * DB * NS * 64 * 16 <= STAGES * STAGEB, "the partial-dQ exchange fits in the stage memory");
  static_assert(2 * DB == KC, "the dQ MFMAs of a tile (2 DB) interleave with its S / dP MFMAs (2 KC)");
};

template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bwd_q_kernel(BwdArgs a) {
  using C = QCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  static_assert(D == 128 || D == 64, "head dims 64 and 128");
  __shared__ __attribute__((aligned(1024))) char smem[C::STAGES * C::STAGEB];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slot = wave & (C::NS - 1);
  const int grp = wave >> 2;  // KV half of each tile; also the ping-pong group
  const int h = lane >> 5, l32 = lane & 31;

  // Work item: (b, hkv, head group, q-tile); the longest causal tiles first.
  const int gp = a.ntiles & 0xff;   // heads per workgroup (set by the launcher)
  const int nqt = a.ntiles >> 8;    // query tiles per head
  const int bmh = 32 * (C::NS / gp);
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = nqt - 1 - (w % nqt);
  int rest = w / nqt;
  const int ngs = p.G / gp;
  const int gs = rest % ngs;
  rest /= ngs;
  const int hk = rest % p.Hkv, b = rest / p.Hkv;
  const int hq = hk * p.G + gs * gp + slot % gp;
  const int m0 = qt * bmh;
  const int mw = m0 + 32 * (slot / gp);  // first query row of this slot
  const int my_m = mw + l32;             // query row of this lane

  // Q / dO rows as MFMA B operands; LSE (log2) and Delta of this lane's row.
  V8 qf[C::KC], df[C::KC];
  float lse2, dlt;
  {
    const int r = min(my_m, p.Sq - 1);
    const T* qs = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh + (int64_t)r * a.q.ss + 8 * h;
    const T* os = (const T*)a.dout.data + b * a.dout.sb + hq * a.dout.sh + (int64_t)r * a.dout.ss + 8 * h;
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      i32x4 x = ld_global16(qs + 16 * kc), y = ld_global16(os + 16 * kc);
      if (my_m >= p.Sq) x = y = i32x4{0, 0, 0, 0};
      qf[kc] = as_v8<V8>(x);
      df[kc] = as_v8<V8>(y);
    }
    const int64_t rr = (int64_t)(b * p.Hq + hq) * p.Sq + r;
    lse2 = a.lse[rr] * kLog2e;
    i32x4 orow[C::KC];
    if (a.delta_out) {
      const T* ob = (const T*)a.o.data + b * a.o.sb + hq * a.o.sh + (int64_t)r * a.o.ss + 8 * h;
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc) orow[kc] = ld_global16(ob + 16 * kc);
      dlt = 0.f;
    } else {
      dlt = a.delta[rr];
    }
    // a row with no allowed key (LSE = -inf) contributes nothing: every one of
    // its pairs is masked, and +inf makes exp2(y - lse2) = 0 for those
    if (!(lse2 > kNegInf)) lse2 = kPosInf;
    // Wait for these loads here, once: without the pins the compiler places a
    // vmcnt(0) wait at their first use inside the tile loop, which would also
    // drain the tile copies in flight on every tile.
    wait_vmcnt<0>();
    if (a.delta_out) {
      // Delta of this lane's row: its half (8 h + 16 kc + t) in fp32, then the
      // other half from lane l ^ 32.
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc) {
        const V8 ov = as_v8<V8>(orow[kc]);
#pragma unroll
        for (int t = 0; t < 8; t += 2) {
          s0 = __builtin_fmaf(to_f32(ov[t]), to_f32(df[kc][t]), s0);
          s1 = __builtin_fmaf(to_f32(ov[t + 1]), to_f32(df[kc][t + 1]), s1);
        }
      }
      const float half = s0 + s1;
      dlt = half + swap_halves(half);
      if (grp == 0 && h == 0 && my_m < p.Sq) a.delta_out[rr] = dlt;
    }
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) {
      pin(qf[kc]);
      pin(df[kc]);
    }
    pin(lse2);
    pin(dlt);
  }
  f32x16 dq[C::DB];
#pragma unroll
  for (int db = 0; db < C::DB; ++db) dq[db] = f32x16{};

  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + bmh);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
  const int t_lo = kv_lo / C::BN;
  const int t_hi = kv_hi > kv_lo ? (kv_hi + C::BN - 1) / C::BN : t_lo;
  const int nt = t_hi - t_lo;

  // Tile copies: tile t_lo + u -> stage u % 4; past the end, redundant copies
  // of the last tile into a free stage keep every wave at 2E per tile.
  const unsigned lds0 = lds_addr_of(smem);
  const T* kp = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh;
  const T* vp = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh;
  int crow[C::E], cchk[C::E];
#pragma unroll
  for (int e = 0; e < C::E; ++e) {
    const int q = (wave * C::E + e) * 64 + lane;
    crow[e] = q / C::CPR;
    cchk[e] = swz_dual_inv<C::CPR>(crow[e], q % C::CPR);
  }
  // Per tile only the scalar bases move; the per-lane byte offsets are
  // recomputed (clamped to row Skv - 1) only for a KV-tail tile.
  int64_t ko[C::E], vo[C::E];
  auto set_offsets = [&](int last) {  // last = Skv - 1 - n0 (clamp)
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int64_t r = min(crow[e], last);
      ko[e] = (r * a.k.ss + cchk[e] * 8) * (int64_t)sizeof(T);
      vo[e] = (r * a.v.ss + cchk[e] * 8) * (int64_t)sizeof(T);
    }
  };
  const int64_t kstep = (int64_t)C::BN * a.k.ss * (int64_t)sizeof(T);
  const int64_t vstep = (int64_t)C::BN * a.v.ss * (int64_t)sizeof(T);
  int ct = t_lo, cst = 0;  // tile the next copy takes, and its stage
  const char* kcur = (const char*)(kp + (int64_t)t_lo * C::BN * a.k.ss);
  const char* vcur = (const char*)(vp + (int64_t)t_lo * C::BN * a.v.ss);
  bool ctail = false;
  auto prep = [&]() {
    const int n0 = ct * C::BN;
    const bool t = n0 + C::BN > p.Skv;
    if (t || ctail) set_offsets(t ? p.Skv - 1 - n0 : C::BN);
    ctail = t;
  };
  set_offsets(C::BN);
  prep();
  // Copies of the next tile in order (past the end the last tile is copied
  // again into the next stage).
  auto issue_next = [&]() {
    const unsigned sb = lds0 + cst * C::STAGEB;
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const unsigned dst = sb + (wave * C::E + e) * 1024;
      load_lds16(kcur + ko[e], dst);
      load_lds16(vcur + vo[e], dst + C::TILEB);
    }
    cst = (cst + 1) & 3;
    if (ct < t_hi - 1) {
      ++ct;
      kcur += kstep;
      vcur += vstep;
      prep();
    }
  };
  auto wait_tile = [&]() { wait_vmcnt<2 * C::E>(); };

  // Lane-constant LDS byte offsets of this wave's KV half: row reads (A
  // operands of S^T / dP^T) and transpose reads of rows r and r + 8 of each
  // 16-row group (A operands of dQ^T).
  const int hrow = 32 * grp;
  int koff[C::KC], voff_lo[C::DB], voff_hi[C::DB];
#pragma unroll
  for (int kc = 0; kc < C::KC; ++kc)
    koff[kc] = (hrow + l32) * C::ROWB + swz_dual<C::CPR>(hrow + l32, 2 * kc + h) * 16;
  {
    const int tr_row = 4 * h + ((lane & 15) >> 2);
    const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
      const int c = 4 * db + (tr_col >> 3), e2 = (tr_col & 7) * 2;
      voff_lo[db] = (hrow + tr_row) * C::ROWB + swz_dual<C::CPR>(hrow + tr_row, c) * 16 + e2;
      voff_hi[db] = (hrow + tr_row + 8) * C::ROWB + swz_dual<C::CPR>(hrow + tr_row + 8, c) * 16 + e2;
    }
  }

  constexpr bool RAW = !SOFTCAP && !ALIBI;
  const float c2 = p.scale_log2;
  const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;

  f32x16 S, DP;  // S^T and dP^T of this wave's 32 KV rows of the current tile
  V8 PS[2];      // packed dS^T of the previous tile (KV rows 0-15, 16-31 of the half)

  // VALU phase: P and dS of the tile at KV row n0 (element r is KV row
  // n0 + hrow + 8(r/4) + 4h + r%4, query row my_m).
  auto vphase = [&](int n0) {
    const int kw = n0 + hrow;  // first KV row of this wave's half
    const bool full = (kw + 32 <= p.Skv) && (!p.causal || kw + 31 <= mw) &&
                      (p.window == 0 || mw + 31 - kw <= p.window);
    int jb = kw + 4 * h;  // pinned: no per-element index is hoisted and kept live
    pin(jb);
    auto form = [&](auto masked) {
      f32x16 de;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float t = 0.f, e;
        const int j = jb + 8 * (r >> 2) + (r & 3);
        if constexpr (RAW) {
          e = fast_exp2(__builtin_fmaf(S[r], c2, -lse2));
        } else {
          const float y = score_log2<SOFTCAP, ALIBI>(S[r], p, slope_log2, my_m, j, t);
          e = fast_exp2(y - lse2);
        }
        if constexpr (decltype(masked)::value) {
          const bool ok = (j < p.Skv) & (!p.causal | (j <= my_m)) & ((p.window == 0) | (my_m - j <= p.window));
          e = ok ? e : 0.f;
        }
        float ds = e * (DP[r] - dlt);
        if constexpr (SOFTCAP) ds *= 1.f - t * t;
        de[r] = ds;
      }
      PS[0] = pack8<T>(de, 0);
      PS[1] = pack8<T>(de, 8);
    };
    if (full)
      form(std::false_type{});
    else
      form(std::true_type{});
    // done before the barrier
    pin(PS[0]);
    pin(PS[1]);
  };

  // MFMA phase: S^T / dP^T of the tile in stage sk (DO_S) and dQ^T of the
  // previous tile in stage sq with PS (DO_Q): a dQ MFMA after every second
  // S / dP MFMA.  Row reads are kept RA MFMAs ahead, transpose reads RB dQ
  // MFMAs ahead.
  auto mphase = [&](auto do_s_c, auto do_q_c, int sk, int sq) {
    constexpr bool DO_S = decltype(do_s_c)::value, DO_Q = decltype(do_q_c)::value;
    const char* sK = smem + sk * C::STAGEB;
    const char* sQ = smem + sq * C::STAGEB;
    auto rdA = [&](int k) {  // k even: K row chunk k/2, odd: V row chunk k/2
      return lds_read16(sK + (k & 1) * C::TILEB + koff[k >> 1]);
    };
    auto rdB = [&](int j, i16x4& lo, i16x4& hi) {
      const int db = j % C::DB, c16 = j / C::DB;
      const char* base = sQ + 16 * c16 * C::ROWB;
      lo = lds_read_tr4(base + voff_lo[db]);
      hi = lds_read_tr4(base + voff_hi[db]);
    };
    constexpr int RA = C::RA, RB = C::RB;
    i32x4 ab[RA + 1];
    i16x4 blo[RB + 1], bhi[RB + 1];
    if constexpr (DO_S) {
#pragma unroll
      for (int k = 0; k < RA; ++k) ab[k] = rdA(k);
      S = f32x16{};
      DP = f32x16{};
    }
    if constexpr (DO_Q) {
#pragma unroll
      for (int j = 0; j < RB; ++j) rdB(j, blo[j], bhi[j]);
    }
#pragma unroll
    for (int k = 0; k < 2 * C::KC; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (DO_S) {
        if (k + RA < 2 * C::KC) ab[(k + RA) % (RA + 1)] = rdA(k + RA);
        if (k & 1) DP = M::mma(as_v8<V8>(ab[k % (RA + 1)]), df[k >> 1], DP);
        else S = M::mma(as_v8<V8>(ab[k % (RA + 1)]), qf[k >> 1], S);
      }
      if constexpr (DO_Q) {
        if (k & 1) {
          const int j = k >> 1;
          if (j + RB < C::KC) rdB(j + RB, blo[(j + RB) % (RB + 1)], bhi[(j + RB) % (RB + 1)]);
          const int db = j % C::DB, c16 = j / C::DB;
          dq[db] = M::mma(cat_tr<V8>(blo[j % (RB + 1)], bhi[j % (RB + 1)]), PS[c16], dq[db]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DO_S) {  // results fixed before the barrier
      pin(S);
      pin(DP);
    }
  };

  // Copies are issued at the start of a VALU phase (the shorter one): a global
  // -> LDS copy holds its wave for tens of cycles at issue.  Tile u + 2 goes
  // to the stage of tile u - 2, whose last reads (dQ of tile u - 2) ended one
  // phase earlier for both halves.
  if (nt > 0) {
    issue_next();  // t_lo
    issue_next();  // t_lo + 1
    wait_tile();
    __syncthreads();
    if (grp) __syncthreads();  // second half starts one phase late
    mphase(std::true_type{}, std::false_type{}, 0, 0);
    __syncthreads();
    for (int u = 0; u + 1 < nt; ++u) {
      issue_next();  // t_lo + u + 2
      vphase((t_lo + u) * C::BN);
      wait_tile();  // tile u + 1 landed
      __syncthreads();
      mphase(std::true_type{}, std::true_type{}, (u + 1) & 3, u & 3);
      __syncthreads();
    }
    vphase((t_hi - 1) * C::BN);
    __syncthreads();
    mphase(std::false_type{}, std::true_type{}, 0, (nt - 1) & 3);
    wait_vmcnt<0>();  // no copy may land after the stages are reused below
    __syncthreads();
    if (!grp) __syncthreads();  // first half: match the second's count
  }

  // dQ = scale * dS K: the second half's partial dQ^T goes through LDS to the
  // first half, which adds it (fixed order) and stores.
  float* xq = (float*)smem + (slot * 64 + lane) * 4;  // 16 B per lane, blocks NS * 1 KB apart
  if (grp) {
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *(f32x4*)(xq + (4 * db + i) * C::NS * 64 * 4) =
            f32x4{dq[db][4 * i], dq[db][4 * i + 1], dq[db][4 * i + 2], dq[db][4 * i + 3]};
  }
  __syncthreads();
  if (!grp && my_m < p.Sq) {
    T* out = (T*)a.dq.data + b * a.dq.sb + hq * a.dq.sh + (int64_t)my_m * a.dq.ss + 4 * h;
    const float sc = p.scale;
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 o = *(const f32x4*)(xq + (4 * db + i) * C::NS * 64 * 4);
        st_global8(out + 32 * db + 8 * i,
                   pack4<T>((dq[db][4 * i] + o[0]) * sc, (dq[db][4 * i + 1] + o[1]) * sc,
                            (dq[db][4 * i + 2] + o[2]) * sc, (dq[db][4 * i + 3] + o[3]) * sc));
      }
  }
}

inline int gqa_pack4(int G) {
  const int gp = G & (-G);
  return gp < 4 ? gp : 4;
}

template <class T, int D>
hipError_t launch_q(const BwdArgs& a, hipStream_t st) {
  using C = QCfg<D>;
  BwdArgs x = a;
  const int gp = gqa_pack4(a.p.G);
  const int bmh = 32 * (C::NS / gp);
  const int nqt = (a.p.Sq + bmh - 1) / bmh;
  x.ntiles = (nqt << 8) | gp;
  const dim3 grid(nqt * (a.p.G / gp) * a.p.B * a.p.Hkv), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  if (sc && al) hipLaunchKernelGGL((bwd_q_kernel<T, D, true, true>), grid, block, 0, st, x);
  else if (sc) hipLaunchKernelGGL((bwd_q_kernel<T, D, true, false>), grid, block, 0, st, x);
  else if (al) hipLaunchKernelGGL((bwd_q_kernel<T, D, false, true>), grid, block, 0, st, x);
  else hipLaunchKernelGGL((bwd_q_kernel<T, D, false, false>), grid, block, 0, st, x);
  return hipGetLastError();
}

#if FLEXATT_D == 128
hipError_t bwd_q_bf16_d128(const BwdArgs& a, hipStream_t st) { return launch_q<__bf16, 128>(a, st); }
hipError_t bwd_q_f16_d128(const BwdArgs& a, hipStream_t st) { return launch_q<_Float16, 128>(a, st); }
#else
hipError_t bwd_q_bf16_d64(const BwdArgs& a, hipStream_t st) { return launch_q<__bf16, 64>(a, st); }
hipError_t bwd_q_f16_d64(const BwdArgs& a, hipStream_t st) { return launch_q<_Float16, 64>(a, st); }
#endif

#endif  // FLEXATT_D == 128 || FLEXATT_D == 64

}  // namespace flexatt

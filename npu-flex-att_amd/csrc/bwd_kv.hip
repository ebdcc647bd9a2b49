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
  static constexpr int STAGES = 8;                     // copies run four tiles ahead
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

  // Tile copies: tile u -> stage u % 8; past the end, redundant copies of the
  // last tile into a free stage keep every wave at 2E + 2 operations per tile.
  const unsigned lds0 = lds_addr_of(smem);
  int crow[C::E], cchk[C::E];  // row / logical chunk of this lane in copy e
#pragma unroll
  for (int e = 0; e < C::E; ++e) {
    const int q = (wave * C::E + e) * 64 + lane;
    crow[e] = q / C::CPR;
    cchk[e] = swz_dual_inv<C::CPR>(crow[e], q % C::CPR);
  }
  // Copies of one tile: E Q rows chunks, E dO chunks and one load of 8 LSE
  // plus 8 Delta values per wave (lanes 0-7 / 8-15), i.e. 2E + 1 operations
  // per wave.  Per tile only scalar bases move; the per-lane offsets are
  // recomputed (clamped to row Sq - 1) only for a query-tail tile.
  const int rl = 8 * wave + (lane & 7);  // LSE / Delta row of this lane's copy
  int64_t cq[C::E], co[C::E];            // per-lane byte offsets, current tile
  int crl;                               // row of the LSE / Delta copy, current tile
  auto set_offsets = [&](int last) {     // last = Sq - 1 - m0 (clamp)
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int64_t r = min(crow[e], last);
      cq[e] = (r * a.q.ss + cchk[e] * 8) * (int64_t)sizeof(T);
      co[e] = (r * a.dout.ss + cchk[e] * 8) * (int64_t)sizeof(T);
    }
    crl = min(rl, last);
  };
  const int64_t qstep = (int64_t)C::BM * a.q.ss * (int64_t)sizeof(T);
  const int64_t ostep = (int64_t)C::BM * a.dout.ss * (int64_t)sizeof(T);
  int is_g = 0, is_qt = qt_lo;  // next tile to copy (head, query tile)
  const char *qcur, *ocur;      // its Q / dO row m0
  const float* lcur;            // its LSE (lanes 0-7) or Delta (lanes 8-15) row m0
  bool tail = false;            // offsets currently clamped
  auto set_head = [&](int g) {
    const int hq = hk * p.G + g;
    const int64_t m0 = (int64_t)qt_lo * C::BM;
    qcur = (const char*)((const T*)a.q.data + b * a.q.sb + hq * a.q.sh + m0 * a.q.ss);
    ocur = (const char*)((const T*)a.dout.data + b * a.dout.sb + hq * a.dout.sh + m0 * a.dout.ss);
    lcur = (lane < 8 ? a.lse : a.delta) + (int64_t)(b * p.Hq + hq) * p.Sq + m0;
  };
  auto prep = [&]() {  // offsets for the tile (is_g, is_qt)
    const int m0 = is_qt * C::BM;
    const bool t = m0 + C::BM > p.Sq;
    if (t || tail) set_offsets(t ? p.Sq - 1 - m0 : C::BM);
    tail = t;
  };
  set_head(0);
  set_offsets(C::BM);
  prep();
  // Copy operation j (0 .. 2E) of the tile going to stage u % 8.
  auto copy_op = [&](int u, int j) {
    const unsigned sb = lds0 + (u & 7) * C::STAGEB;
    if (j < C::E) {
      load_lds16(qcur + cq[j], sb + (wave * C::E + j) * 1024);
    } else if (j < 2 * C::E) {
      load_lds16(ocur + co[j - C::E], sb + C::TILEB + (wave * C::E + j - C::E) * 1024);
    } else if (lane < 16) {
      load_lds4(lcur + crl, sb + 2 * C::TILEB + 64 * wave);
    }
  };
  // Move to the next tile to copy (past the end the last tile is copied again).
  auto advance = [&]() {
    if (is_g < p.G - 1 || is_qt < qt_lo + nqt - 1) {
      if (++is_qt == qt_lo + nqt) {
        is_qt = qt_lo;
        set_head(++is_g);
      } else {
        qcur += qstep;
        ocur += ostep;
        lcur += C::BM;
      }
      prep();
    }
  };
  auto issue = [&](int u) {
#pragma unroll
    for (int j = 0; j <= 2 * C::E; ++j) copy_op(u, j);
    advance();
  };

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

  // Two register sets alternate between pipeline iterations (no copies):
  // iteration u reads S / dP of tile u and packed P / dS of tile u-1 from its
  // current set, and writes S / dP of tile u+1 and P / dS of tile u to the
  // other set.
  struct Set {
    f32x16 S, DP;
    V8 PP[C::NPK], PS[C::NPK];
  };
  Set s0, s1;

  // LSE and Delta of this lane's 16 query rows of the tile in stage st
  // (stored per 8 rows: 8 LSE values, then 8 Delta values).
  f32x4 L4[4], D4[4];
  auto read_rows = [&](int st) {
    const float* sR = (const float*)(smem + st * C::STAGEB + 2 * C::TILEB);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      L4[i] = __builtin_bit_cast(f32x4, lds_read16(sR + 16 * i + 4 * h));
      D4[i] = __builtin_bit_cast(f32x4, lds_read16(sR + 16 * i + 8 + 4 * h));
    }
  };

  // Which tiles need the per-element pass, for this wave's KV rows
  // [kw0, kw0 + 32): query tail, KV tail, causal diagonal, window edge.
  auto need_mask = [&](int m0) {
    return (m0 + C::BM > p.Sq) || (kw0 + 32 > p.Skv) || (p.causal && m0 < kw0 + 31) ||
           (p.window > 0 && m0 + C::BM - 1 - kw0 > p.window);
  };

  int cg = 0, cqt = qt_lo;  // tile whose P / dS is formed next (head, query tile)
  auto tile_info = [&](int& m0, float& slope) {
    const int hq = hk * p.G + cg;
    m0 = cqt * C::BM;
    slope = ALIBI ? p.alibi[hq] * kLog2e : 0.f;
    if (++cqt == qt_lo + nqt) {
      cqt = qt_lo;
      ++cg;
    }
  };

  // P and log2-domain transform of element r (query row m0 + 8(r/4) + 4h +
  // r%4, KV row my_kv); t = tanh for the soft-cap derivative.
  auto p_elem = [&](const Set& x, int r, int m0, float sl, float& t) {
    const float l2 = L4[r >> 2][r & 3] * kLog2e;
    float sv = x.S[r];
    pin(sv);  // read from the accumulator here, not hoisted into an earlier step
    if constexpr (RAW) {
      t = 0.f;
      return fast_exp2(__builtin_fmaf(sv, c2, -l2));
    } else {
      const int q = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
      const float y = score_log2<SOFTCAP, ALIBI>(sv, p, sl, q, my_kv, t);
      return fast_exp2(y - l2);
    }
  };

  // Masked recompute of P / dS of the tile in `cur` into `nxt` (rare).
  auto valu_masked = [&](const Set& cur, int m0, float sl, Set& nxt) {
    f32x16 pe, de;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
      float t;
      float e = p_elem(cur, r, m0, sl, t);
      const bool ok = (q < p.Sq) & (my_kv < p.Skv) & (!p.causal | (my_kv <= q)) &
                      ((p.window == 0) | (q - my_kv <= p.window));
      e = ok ? e : 0.f;
      float ds = e * (cur.DP[r] - D4[r >> 2][r & 3]);
      if constexpr (SOFTCAP) ds *= 1.f - t * t;
      pe[r] = e;
      de[r] = ds;
    }
    nxt.PP[0] = pack8<T>(pe, 0);
    nxt.PP[1] = pack8<T>(pe, 8);
    nxt.PS[0] = pack8<T>(de, 0);
    nxt.PS[1] = pack8<T>(de, 8);
#pragma unroll
    for (int i = 0; i < C::NPK; ++i) {  // kept inside the branch
      pin(nxt.PP[i]);
      pin(nxt.PS[i]);
    }
  };

  // Row reads (A operands of S / dP) of the tile in stage st, MFMA k.
  auto rdA = [&](int st, int k) {
    const char* base = smem + st * C::STAGEB + (k & 1) * C::TILEB;
    return lds_read16(base + koff[k >> 1]);
  };
  // Transpose reads (A operands of dV / dK) of the tile in stage st, MFMA j.
  auto rdB = [&](int st, int j, i16x4& lo, i16x4& hi) {
    const int db = (j >> 1) % C::DB, qc = (j >> 1) / C::DB;
    const char* base = smem + st * C::STAGEB + ((j & 1) ? 0 : C::TILEB) + 16 * qc * C::ROWB;
    lo = lds_read_tr4(base + voff_lo[db]);
    hi = lds_read_tr4(base + voff_hi[db]);
  };
  auto mfma_kv = [&](int j, i16x4 lo, i16x4 hi, const Set& x) {
    const int db = (j >> 1) % C::DB, qc = (j >> 1) / C::DB;
    if (j & 1) dk[db] = M::mma(cat_tr<V8>(lo, hi), x.PS[qc], dk[db]);
    else dv[db] = M::mma(cat_tr<V8>(lo, hi), x.PP[qc], dv[db]);
  };

  // S / dP of the tile in stage st into x (fills the pipeline).
  auto fill = [&](int st, Set& x) {
    i32x4 ab[5];
#pragma unroll
    for (int k = 0; k < 4; ++k) ab[k] = rdA(st, k);
    x.S = f32x16{};
    x.DP = f32x16{};
#pragma unroll
    for (int k = 0; k < 2 * C::KC; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      if (k + 4 < 2 * C::KC) ab[(k + 4) % 5] = rdA(st, k + 4);
      if (k & 1) x.DP = M::mma(as_v8<V8>(ab[k % 5]), vreg[k >> 1], x.DP);
      else x.S = M::mma(as_v8<V8>(ab[k % 5]), kreg[k >> 1], x.S);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // dV / dK of the tile in stage st with the packed P / dS of x (drains it).
  auto drain = [&](int st, const Set& x) {
    i16x4 blo[3], bhi[3];
    rdB(st, 0, blo[0], bhi[0]);
    rdB(st, 1, blo[1], bhi[1]);
#pragma unroll
    for (int j = 0; j < 4 * C::DB; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      if (j + 2 < 4 * C::DB) rdB(st, j + 2, blo[(j + 2) % 3], bhi[(j + 2) % 3]);
      mfma_kv(j, blo[j % 3], bhi[j % 3], x);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  constexpr int CNT = 2 * C::E + 1;  // copy operations per tile per wave

  // One pipeline iteration: the 16 S / dP MFMAs of tile u+1 (row reads four
  // ahead), then the 16 dV / dK MFMAs of tile u-1 (transpose reads two
  // ahead); every MFMA step carries half of one element of tile u's P / dS.
  auto step = [&](int u, Set& cur, Set& nxt) {
    wait_vmcnt<2 * CNT>();
    __syncthreads();  // tile u+1 landed; stage (u - 4) % 8 no longer read
    int m0;
    float sl;
    tile_info(m0, sl);
    const int sn = (u + 1) & 7, sc = u & 7, sp = (u > 0 ? u - 1 : 0) & 7;
    read_rows(sc);
    i32x4 ab[5];
#pragma unroll
    for (int k = 0; k < 4; ++k) ab[k] = rdA(sn, k);
    i16x4 blo[3], bhi[3];
    nxt.S = f32x16{};
    nxt.DP = f32x16{};
    f32x16 pe, de;
    float tt[16];
    constexpr int NA = 2 * C::KC, NBK = 4 * C::DB;
#pragma unroll
    for (int k = 0; k < NA + NBK; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      if (k + 4 < NA) ab[(k + 4) % 5] = rdA(sn, k + 4);
      if (k >= 1 && k <= 2 * C::E + 1) copy_op(u + 4, k - 1);  // copies of tile u+4
      if (k >= NA - 2 && k - (NA - 2) < NBK) {
        const int j = k - (NA - 2);
        rdB(sp, j, blo[j % 3], bhi[j % 3]);
      }
      if (k < NA) {
        if (k & 1) nxt.DP = M::mma(as_v8<V8>(ab[k % 5]), vreg[k >> 1], nxt.DP);
        else nxt.S = M::mma(as_v8<V8>(ab[k % 5]), kreg[k >> 1], nxt.S);
      } else {
        const int j = k - NA;
        mfma_kv(j, blo[j % 3], bhi[j % 3], cur);
      }
      const int r = k >> 1;
      if (!(k & 1)) {
        float t;
        float e = p_elem(cur, r, m0, sl, t);
        pin(e);  // formed in this step (not sunk below the MFMA run)
        pe[r] = e;
        tt[r] = t;
      } else {
        float dpv = cur.DP[r];
        pin(dpv);
        float ds = pe[r] * (dpv - D4[r >> 2][r & 3]);
        if constexpr (SOFTCAP) ds *= 1.f - tt[r] * tt[r];
        pin(ds);
        de[r] = ds;
        if (r == 7) {
          nxt.PP[0] = pack8<T>(pe, 0);
          nxt.PS[0] = pack8<T>(de, 0);
          pin(nxt.PP[0]);
          pin(nxt.PS[0]);
        } else if (r == 15) {
          nxt.PP[1] = pack8<T>(pe, 8);
          nxt.PS[1] = pack8<T>(de, 8);
          pin(nxt.PP[1]);
          pin(nxt.PS[1]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    advance();
#pragma unroll
    for (int i = 0; i < C::NPK; ++i) {  // fast path computed before the branch
      pin(nxt.PP[i]);
      pin(nxt.PS[i]);
    }
    if (need_mask(m0)) valu_masked(cur, m0, sl, nxt);
  };

  if (ntile > 0) {
    issue(0);
    issue(1);
    issue(2);
    issue(3);
    wait_vmcnt<3 * CNT>();
    __syncthreads();
    fill(0, s0);
#pragma unroll
    for (int i = 0; i < C::NPK; ++i) {  // dV / dK of "tile -1" add zero
      s0.PP[i] = V8{};
      s0.PS[i] = V8{};
    }
    int u = 0;
    for (; u + 2 <= ntile; u += 2) {
      step(u, s0, s1);
      step(u + 1, s1, s0);
    }
    if (u < ntile) {
      step(u, s0, s1);
      drain((ntile - 1) & 7, s1);
    } else {
      drain((ntile - 1) & 7, s0);
    }
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

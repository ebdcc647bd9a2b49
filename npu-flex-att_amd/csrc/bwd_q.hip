// Flash-attention backward dQ for fp16/bf16 on gfx950 MFMA (query-stationary
// tile stream).
//
// Semantics: npu_flash_attention.py:298-402 (flash_attn_bwd_dq_kernel): P is
// recomputed from the forward LSE (including the ALiBi bias, which the
// reference's backward kernels omit), dP = dO V^T,
// dS = P (dP - Delta) scale (1 - tanh^2), dQ = dS K; dS is rounded to the
// input dtype before its MFMA, as the reference does before tl.dot.
//
// Decomposition
//  * One workgroup = 4 waves (one per SIMD, the whole register file each) =
//    one (batch, KV head), gp query heads that share it (gp = the largest power
//    of two dividing G, at most 4) and 32 * 4 / gp query rows of each.  Each
//    wave owns 32 query rows of one head and each lane one query row: its Q
//    and dO rows stay in registers as MFMA B operands and its LSE and Delta
//    are one scalar each.
//  * S^T = K Q^T and dP^T = V dO^T per 32-row block of a 64-row KV tile (A =
//    K / V rows from LDS); dQ^T += K^T dS^T with K^T read by the LDS transpose
//    read, so the K tile is read both ways (dual-use swizzle).
//  * K / V tiles are copied global -> LDS with direct-to-LDS loads two tiles
//    ahead into four stages, one barrier per tile.
//  * Software pipeline inside each wave, each step in a fixed order: the S^T
//    MFMAs of tile t, then its dP^T MFMAs with P = exp2(y - LSE) formed in
//    their shadow, then the dQ MFMAs of tile t-1 with dS of tile t formed in
//    theirs.
//  * Tiles that cross the causal diagonal, the window edge or the KV tail for
//    some row of a wave take the fast path first and then recompute dS with
//    the per-element mask (only the packed dS registers differ between the
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
struct QCfg {
  static constexpr int NW = 4;       // waves per workgroup, one per SIMD
  static constexpr int BN = 64;      // KV rows per tile
  static constexpr int NB = BN / 32;
  static constexpr int KC = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int CPR = D / 8;
  static constexpr int ROWB = 2 * D;
  static constexpr int TILEB = BN * ROWB;         // one of K / V
  static constexpr int E = TILEB / (1024 * NW);   // 1 KB copies per wave per tensor
  static constexpr int STAGEB = 2 * TILEB;
  static constexpr int STAGES = 4;
  static constexpr int NPK = 2 * NB;              // packed dS operands per tile
  static_assert(E * 1024 * NW == TILEB, "tile must split into 1 KB copies");
};

template <class T, int D, bool SOFTCAP, bool ALIBI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void bwd_q_kernel(BwdArgs a) {
  using C = QCfg<D>;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  static_assert(C::NB == 2 && C::KC == 8 && C::DB == 4, "the hand-ordered step assumes D = 128, 64-row tiles");
  __shared__ __attribute__((aligned(1024))) char smem[C::STAGES * C::STAGEB];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;

  // Work item: (b, hkv, head group, q-tile); the longest causal tiles first.
  const int gp = a.ntiles & 0xff;   // heads per workgroup (set by the launcher)
  const int nqt = a.ntiles >> 8;    // query tiles per head
  const int bmh = 32 * (C::NW / gp);
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = nqt - 1 - (w % nqt);
  int rest = w / nqt;
  const int ngs = p.G / gp;
  const int gs = rest % ngs;
  rest /= ngs;
  const int hk = rest % p.Hkv, b = rest / p.Hkv;
  const int hq = hk * p.G + gs * gp + wave % gp;
  const int m0 = qt * bmh;
  const int mw = m0 + 32 * (wave / gp);  // first query row of this wave
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
    dlt = a.delta[rr];
    // a row with no allowed key (LSE = -inf) contributes nothing: every one of
    // its pairs is masked, and +inf makes exp2(y - lse2) = 0 for those
    if (!(lse2 > kNegInf)) lse2 = kPosInf;
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
  int ct = t_lo;  // tile the next issue() copies
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
  // issue(u) copies tile t_lo + u into stage u % 4 (calls come in order of u;
  // past the end the last tile is copied again).
  auto issue = [&](int u) {
    const unsigned sb = lds0 + (u & 3) * C::STAGEB;
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const unsigned dst = sb + (wave * C::E + e) * 1024;
      load_lds16(kcur + ko[e], dst);
      load_lds16(vcur + vo[e], dst + C::TILEB);
    }
    if (ct < t_hi - 1) {
      ++ct;
      kcur += kstep;
      vcur += vstep;
      prep();
    }
  };
  auto wait_tile = [&]() { wait_vmcnt<2 * C::E>(); };

  // Lane-constant LDS byte offsets (row reads, and transpose reads of rows
  // r and r + 8 of each 16-row group).
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
  const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;

  // Tiles [tm_lo, tm_hi) are fully allowed for every row of this wave.
  int tm_hi = p.Skv / C::BN;
  if (p.causal) tm_hi = min(tm_hi, (mw + 1) / C::BN);
  int tm_lo = 0;
  if (p.window > 0) tm_lo = max(0, (mw + 31 - p.window + C::BN - 1) / C::BN);
  tm_hi = __builtin_amdgcn_readfirstlane(tm_hi);
  tm_lo = __builtin_amdgcn_readfirstlane(tm_lo);

  f32x16 S[C::NB], DP[C::NB];  // S^T and dP^T of the tile being processed
  f32x16 PE[C::NB];            // P^T of that tile
  V8 PS[C::NPK];               // packed dS^T of the previous tile

  // Element r of block bb of the current tile (KV row n0 + 32bb + 8(r/4) +
  // 4h + r%4, query row my_m): P, and t = tanh for the soft-cap derivative.
  auto p_elem = [&](int bb, int r, int n0, float& t) {
    if constexpr (RAW) {
      t = 0.f;
      return fast_exp2(__builtin_fmaf(S[bb][r], c2, -lse2));
    } else {
      const int j = n0 + 32 * bb + 8 * (r >> 2) + 4 * h + (r & 3);
      const float y = score_log2<SOFTCAP, ALIBI>(S[bb][r], p, slope_log2, my_m, j, t);
      return fast_exp2(y - lse2);
    }
  };
  float TT[C::NB][16];  // tanh values (soft-cap only; unused otherwise)
  auto ds_elem = [&](int bb, int r) {
    float ds = PE[bb][r] * (DP[bb][r] - dlt);
    if constexpr (SOFTCAP) ds *= 1.f - TT[bb][r] * TT[bb][r];
    return ds;
  };
  // Masked recompute of dS for a tile that needs the per-element mask.
  auto ds_masked = [&](int n0, V8 (&ps)[C::NPK]) {
#pragma unroll
    for (int bb = 0; bb < C::NB; ++bb) {
      f32x16 de;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = n0 + 32 * bb + 8 * (r >> 2) + 4 * h + (r & 3);
        const bool ok = (j < p.Skv) & (!p.causal | (j <= my_m)) & ((p.window == 0) | (my_m - j <= p.window));
        const float ds = ds_elem(bb, r);
        de[r] = ok ? ds : 0.f;
      }
      ps[2 * bb] = pack8<T>(de, 0);
      ps[2 * bb + 1] = pack8<T>(de, 8);
    }
    // results fixed inside the (rarely taken) branch, so that the compiler
    // keeps it a branch instead of computing it on every tile and selecting
#pragma unroll
    for (int i = 0; i < C::NPK; ++i) pin(ps[i]);
  };

  // Region A1 + A2 for the tile in stage st: S^T MFMAs (row reads of K four
  // ahead), then dP^T MFMAs (row reads of V four ahead) with P formed in
  // their shadow.
  auto regions_a = [&](int st, int n0) {
    const char* sK = smem + st * C::STAGEB;
    const char* sV = sK + C::TILEB;
    constexpr int NA = C::NB * C::KC;  // 16
    auto rdK = [&](int k) { return lds_read16(sK + (k & 1) * 32 * C::ROWB + koff[k >> 1]); };
    auto rdV = [&](int k) { return lds_read16(sV + (k & 1) * 32 * C::ROWB + koff[k >> 1]); };
    i32x4 ab[5];
#pragma unroll
    for (int k = 0; k < 4; ++k) ab[k] = rdK(k);
#pragma unroll
    for (int bb = 0; bb < C::NB; ++bb) {
      S[bb] = f32x16{};
      DP[bb] = f32x16{};
    }
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      if (k + 4 < NA) ab[(k + 4) % 5] = rdK(k + 4);
      else ab[(k + 4) % 5] = rdV(k + 4 - NA);
      S[k & 1] = M::mma(as_v8<V8>(ab[k % 5]), qf[k >> 1], S[k & 1]);
    }
    // the read ring continues: V read k sits at ring position (NA + k) % 5
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      if (k + 4 < NA) ab[(NA + k + 4) % 5] = rdV(k + 4);
      DP[k & 1] = M::mma(as_v8<V8>(ab[(NA + k) % 5]), df[k >> 1], DP[k & 1]);
      // two elements of P per MFMA (both S^T blocks are complete by now)
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int idx = 2 * k + x, bb = idx >> 4, r = idx & 15;
        float t;
        PE[bb][r] = p_elem(bb, r, n0, t);
        if constexpr (SOFTCAP) TT[bb][r] = t;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Region B: dQ^T MFMAs of the tile in stage sp with PS (transpose reads of K
  // two ahead); after MFMA k, two elements of the current tile's dS.
  auto region_b = [&](int sp, bool do_ds, V8 (&psn)[C::NPK]) {
    const char* sKp = smem + sp * C::STAGEB;
    constexpr int NBQ = C::DB * C::NPK;  // 16
    auto rdB = [&](int k, i16x4& lo, i16x4& hi) {
      const int db = k % C::DB, c16 = k / C::DB;  // 16-row KV chunk
      const char* base = sKp + 16 * c16 * C::ROWB;
      lo = lds_read_tr4(base + voff_lo[db]);
      hi = lds_read_tr4(base + voff_hi[db]);
    };
    i16x4 blo[3], bhi[3];
    rdB(0, blo[0], bhi[0]);
    rdB(1, blo[1], bhi[1]);
    f32x16 de[C::NB];
#pragma unroll
    for (int k = 0; k < NBQ; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      if (k + 2 < NBQ) rdB(k + 2, blo[(k + 2) % 3], bhi[(k + 2) % 3]);
      const int db = k % C::DB, c16 = k / C::DB;
      dq[db] = M::mma(cat_tr<V8>(blo[k % 3], bhi[k % 3]), PS[c16], dq[db]);
      if (do_ds) {
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int idx = 2 * k + x, bb = idx >> 4, r = idx & 15;
          de[bb][r] = ds_elem(bb, r);
          if (r == 15) {
            psn[2 * bb] = pack8<T>(de[bb], 0);
            psn[2 * bb + 1] = pack8<T>(de[bb], 8);
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  if (nt > 0) {
    issue(0);
    issue(1);
    {
      wait_tile();
      __syncthreads();
      issue(2);
      const int n0 = t_lo * C::BN;
      regions_a(0, n0);
#pragma unroll
      for (int bb = 0; bb < C::NB; ++bb) {
        f32x16 de;
#pragma unroll
        for (int r = 0; r < 16; ++r) de[r] = ds_elem(bb, r);
        PS[2 * bb] = pack8<T>(de, 0);
        PS[2 * bb + 1] = pack8<T>(de, 8);
      }
      if (t_lo < tm_lo || t_lo >= tm_hi) ds_masked(n0, PS);
    }
    for (int u = 1; u < nt; ++u) {
      wait_tile();
      __syncthreads();  // tile u landed; stage (u - 2) % 4 no longer read
      issue(u + 2);
      const int t = t_lo + u, n0 = t * C::BN;
      regions_a(u & 3, n0);
      V8 PSn[C::NPK];
      region_b((u - 1) & 3, true, PSn);
#pragma unroll
      for (int i = 0; i < C::NPK; ++i) pin(PSn[i]);  // fast path computed before the branch
      if (t < tm_lo || t >= tm_hi) ds_masked(n0, PSn);
#pragma unroll
      for (int i = 0; i < C::NPK; ++i) PS[i] = PSn[i];
    }
    V8 unused[C::NPK];
    region_b((nt - 1) & 3, false, unused);
    wait_vmcnt<0>();  // redundant copies in flight must land before the workgroup ends
  }

  // dQ = scale * dS K (dQ^T accumulated: lane = query row, 4 consecutive d).
  if (my_m < p.Sq) {
    T* out = (T*)a.dq.data + b * a.dq.sb + hq * a.dq.sh + (int64_t)my_m * a.dq.ss + 4 * h;
    const float sc = p.scale;
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st_global8(out + 32 * db + 8 * i, pack4<T>(dq[db][4 * i] * sc, dq[db][4 * i + 1] * sc,
                                                  dq[db][4 * i + 2] * sc, dq[db][4 * i + 3] * sc));
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
  const int bmh = 32 * (C::NW / gp);
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

hipError_t bwd_q_bf16_d128(const BwdArgs& a, hipStream_t st) { return launch_q<__bf16, 128>(a, st); }
hipError_t bwd_q_f16_d128(const BwdArgs& a, hipStream_t st) { return launch_q<_Float16, 128>(a, st); }

#endif  // FLEXATT_D == 128

}  // namespace flexatt

// Flash-attention forward at D = 256 for fp16/bf16 on gfx950 MFMA, with
// wave-specialised pairs.
//
// Semantics: npu_flash_attention.py:17-166 (flash_attn_fwd_kernel), as in
// fwd_mfma.hip: online softmax over KV tiles, O in the input dtype, LSE in
// fp32 natural log, the score order scale -> soft-cap -> ALiBi -> mask, GQA
// head h -> h / G.
//
// Why a second D = 256 form: 32 query rows of O at D = 256 are 128
// accumulator registers, and with their Q rows (64) a wave that does both
// the scores and the PV products fits only one wave per SIMD, which then
// cannot overlap its softmax with its MFMAs.  Here the two jobs are split
// over the two waves of a SIMD:
//  * One workgroup = 8 waves = four pairs; pair p (waves p and p + 4, on one
//    SIMD) owns 32 query rows of one head of the (batch, KV head) group
//    (gp heads per workgroup, as in fwd_mfma.hip).
//  * The S-wave (p) holds the Q rows (MFMA B operands) and computes
//    S^T = K Q^T for a 64-key tile (32 MFMAs, K rows from LDS), then the
//    softmax: mask, row max, lazy rescale, P = exp2(y - m), row sums.  It
//    hands P (packed, as the PV B operands) and the per-row rescale factor
//    alpha (1 unless the running max moved) to its partner through LDS.
//  * The PV-wave (p + 4) holds O^T in registers, rescales it by alpha when
//    some row's max moved, and runs O^T += V^T P^T (32 MFMAs, V^T from the
//    LDS transpose read).  It issues every tile copy.
//  * Step u has two phases separated by workgroup barriers:
//      M(u): S-wave: the S^T MFMAs of tile u;  PV-wave: the copy of V tile
//            u, the packed P / alpha of tile u-1 and its first transpose
//            reads;
//      V(u): S-wave: the softmax of tile u, into the exchange buffer;
//            PV-wave: the PV MFMAs of tile u-1, the copy of K tile u+2, then
//            the wait for K tile u+1 and V tile u;
//    so each SIMD alternates between the S-wave's MFMAs and the PV-wave's
//    MFMAs beside the S-wave's VALU work.
//  * K and V live in rings of two 32 KB slots each: the K slot of tile u is
//    free once M(u) ends, the V slot of tile u-2 once V(u-1) ends, so each
//    copy has about one step to land.  (The 32-key form, a tuning override,
//    has rings of four 16 KB slots, two exchange buffers and all copies in
//    M(u): K tile u+3, V tile u+2.)  Tiles are unpadded with the per-row
//    chunk swizzles of fwd_mfma.hip (swz_col for K, swz_tr for V).
//  * The lazy rescale, the interval masks and the mask-free interior tiles
//    are those of fwd_mfma.hip; O leaves through a per-pair LDS tile as
//    16-byte row-contiguous stores.
//  * Block-sparse maps (BLK): the workgroup walks only the KV tiles whose
//    128 x 128 block is computed for some pair (a list built in LDS at the
//    start, as fwd_mfma.hip); in a listed tile, an S-wave whose own block is
//    removed skips its MFMAs and hands P = 0, alpha = 1 to its partner.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

#if FLEXATT_D == 256

struct WsCfg {
  static constexpr int D = 256;
  static constexpr int NP = 4;                    // wave pairs, one per SIMD
  static constexpr int NW = 2 * NP;
#ifdef FLEXATT_WS_BN
  static constexpr int BN = FLEXATT_WS_BN;        // tuning override (32 or 64)
#else
  static constexpr int BN = 64;                   // keys per tile (12-17% faster than 32)
#endif
  static constexpr int NB = BN / 32;              // 32-key blocks per tile
  static constexpr int KC = D / 16;               // k chunks of S^T
  static constexpr int DB = D / 32;               // 32-row blocks of O^T
  static constexpr int CPR = D / 8;               // 16-byte chunks per row
  static constexpr int ROWB = 2 * D;              // bytes per row
  static constexpr int TILEB = BN * ROWB;         // one K or V tile (16 KB)
  static constexpr int E = TILEB / (1024 * NP);   // 1 KB copies per PV-wave per tile
  // ring slots of K and of V: four 16 KB slots for 32-key tiles, two 32 KB
  // slots for 64-key tiles (copy schedules below)
  static constexpr int SLOTS = BN == 32 ? 4 : 2;
  static constexpr int KOFF = 0, VOFF = SLOTS * TILEB;
  static constexpr int XP = 2 * NB * 1024;        // per pair: P (2 NB operands of 1 KB), then alpha (64 floats)
  static constexpr int XPAIR = XP + 256;
  // exchange buffers: two for 32-key tiles; one for 64-key tiles, which is
  // enough because the barrier that starts V(u) (where P(u) is written)
  // waits for every wave's LDS reads of P(u-1), issued in M(u)
  static constexpr int NX = BN == 32 ? 2 : 1;
  static constexpr int XOFF = 2 * SLOTS * TILEB;
  static constexpr int LDSB = XOFF + NX * NP * XPAIR;
  static constexpr int RA = 4;                    // PV-wave: transpose reads this many MFMAs ahead
  static_assert((BN == 32 || BN == 64) && E * 1024 * NP == TILEB && LDSB <= 160 * 1024, "LDS layout");
  static_assert(SLOTS * TILEB >= NP * 32 * ROWB, "O leaves through the K ring");
};

constexpr float kWsRescaleThreshold = 8.0f;  // log2 units (as fwd_mfma.hip)

template <class T, bool SOFTCAP, bool ALIBI, bool BLK>
__global__ __launch_bounds__(WsCfg::NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fwd_ws_kernel(FwdArgs a) {
  using C = WsCfg;
  using M = Mfma<T>;
  using V8 = typename M::v8;
  __shared__ __attribute__((aligned(1024))) char smem[C::LDSB];

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pr = wave & (C::NP - 1);
  const bool s_wave = wave < C::NP;
  const int h = lane >> 5, l32 = lane & 31;

  // Work item: (b, hkv, head group, q-tile), as fwd_mfma.hip.
  const int gp = a.gpack;
  const int bmh = 32 * (C::NP / gp);  // query rows per head
  const int ngs = p.G / gp;
  int kq, rest;
  if (!xcd_lpt_item(blockIdx.x, a.nqt, ngs * p.B * p.Hkv, kq, rest)) {
    const int w = xcd_remap(blockIdx.x, gridDim.x);
    kq = w % a.nqt;
    rest = w / a.nqt;
  }
  const int qt = a.nqt - 1 - kq;
  const int gs = rest % ngs;
  rest /= ngs;
  const int hk = rest % p.Hkv, b = rest / p.Hkv;
  const int hq = hk * p.G + gs * gp + pr % gp;
  const int m0 = qt * bmh;
  const int mw = m0 + 32 * (pr / gp);  // first query row of this pair
  const int my_m = mw + l32;

  // KV range of the workgroup's rows: causal, window, document bounds.
  int kv_lo = 0, kv_hi = p.Skv;
  if (p.causal) kv_hi = min(kv_hi, m0 + bmh);
  if (p.window > 0) kv_lo = max(0, m0 - p.window);
  if (p.doc) {
    int l0, h0, l1, h1;
    doc_bounds(p, b, min(m0, p.Sq - 1), l0, h0);
    doc_bounds(p, b, min(m0 + bmh, p.Sq) - 1, l1, h1);
    kv_lo = max(kv_lo, l0);
    kv_hi = min(kv_hi, h1);
  }
  const int t_lo = kv_lo / C::BN;
  const int t_hi = (kv_hi + C::BN - 1) / C::BN;
  int nv = max(t_hi - t_lo, 0);  // tiles walked

  // Block-sparse maps: each pair's row of the block map over the
  // workgroup's KV range, then the list of the tiles whose block is computed
  // for some pair (walk position v -> tile tile_of(v)), in dynamic LDS.
  extern __shared__ unsigned char sblk[];
  __shared__ int s_nv;
  const int bstride = a.bstride;
  unsigned short* tlist = (unsigned short*)(sblk + C::NP * bstride);
  const int kb_base = t_lo * C::BN / kBlk;
  if (BLK && nv > 0) {
    if (s_wave) {
      const unsigned char* row = block_row(p, b, hq, min(mw, p.Sq - 1));
      const int nkb = (t_hi * C::BN - 1) / kBlk - kb_base + 1;
      for (int i = lane; i < nkb; i += 64) sblk[pr * bstride + i] = row[kb_base + i];
    }
    __syncthreads();
    if (wave == 0) {
      int base = 0;
      for (int t0 = t_lo; t0 < t_hi; t0 += 64) {
        const int t = t0 + lane;
        bool live = false;
        if (t < t_hi) {
          const int kb = t * C::BN / kBlk - kb_base;
#pragma unroll
          for (int w = 0; w < C::NP; ++w) live = live || sblk[w * bstride + kb] != 0;
        }
        const unsigned long long m = __builtin_amdgcn_ballot_w64(live);
        if (live) tlist[base + __builtin_popcountll(m & ((1ull << lane) - 1))] = (unsigned short)(t - t_lo);
        base += __builtin_popcountll(m);
      }
      if (lane == 0) s_nv = base;
    }
    __syncthreads();
    nv = __builtin_amdgcn_readfirstlane(s_nv);
  }
  auto tile_of = [&](int v) -> int {
    if constexpr (BLK) return t_lo + __builtin_amdgcn_readfirstlane((int)tlist[v]);
    else return t_lo + v;
  };

  // exchange buffer of tile u: this pair's P operands and alpha
  auto xp = [&](int u) { return smem + C::XOFF + (u % C::NX) * (C::NP * C::XPAIR) + pr * C::XPAIR; };

  if (s_wave) {
    // ========================= S-wave: S^T, softmax ==========================
    const T* qp = (const T*)a.q.data + b * a.q.sb + hq * a.q.sh;
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
    // This lane's row attends to the keys [row_lo, row_lo + row_w).
    int dlo, dhi;
    doc_bounds(p, b, min(my_m, p.Sq - 1), dlo, dhi);
    int row_lo = max(dlo, 0), row_hi = min(dhi, p.Skv);
    if (p.causal) row_hi = min(row_hi, my_m + 1);
    if (p.window > 0) row_lo = max(row_lo, my_m - p.window);
    const unsigned row_w = (unsigned)max(row_hi - row_lo, 0);
    // Tiles [tm_lo, tm_hi) are fully allowed for every row of the pair.
    int tm_hi = p.Skv / C::BN;
    if (p.causal) tm_hi = min(tm_hi, (mw + 1) / C::BN);
    int tm_lo = 0;
    if (p.window > 0) tm_lo = max(0, (mw + 31 - p.window + C::BN - 1) / C::BN);
    if (p.doc) {
      int l0, h0, l1, h1;
      doc_bounds(p, b, min(mw, p.Sq - 1), l0, h0);
      doc_bounds(p, b, min(mw + 31, p.Sq - 1), l1, h1);
      tm_lo = max(tm_lo, (l1 + C::BN - 1) / C::BN);
      tm_hi = min(tm_hi, h0 / C::BN);
      if (tm_hi < tm_lo) tm_hi = tm_lo;
    }
    tm_hi = __builtin_amdgcn_readfirstlane(tm_hi);
    tm_lo = __builtin_amdgcn_readfirstlane(tm_lo);

    constexpr bool RAW = !SOFTCAP && !ALIBI;
    float c2 = p.scale_log2;
    if constexpr (RAW) {
      if (c2 < 0.f) {  // a negative scale moves into the sign of Q (exact)
#pragma unroll
        for (int kc = 0; kc < C::KC; ++kc)
          qf[kc] = as_v8<V8>(__builtin_bit_cast(i32x4, qf[kc]) ^ i32x4{(int)0x80008000, (int)0x80008000,
                                                                       (int)0x80008000, (int)0x80008000});
        c2 = -c2;
      }
      if (c2 == 0.f) c2 = 1e-30f;
    }
    const float slope_log2 = ALIBI ? p.alibi[hq] * kLog2e : 0.f;
    int koff[C::KC];
#pragma unroll
    for (int kc = 0; kc < C::KC; ++kc) koff[kc] = l32 * C::ROWB + swz_col<C::CPR>(l32, 2 * kc + h) * 16;
    float m_run = kNegInf, l_run = 0.f;

    __syncthreads();  // prologue: K tile 0 landed
    for (int u = 0; u <= nv; ++u) {
      const bool act = u < nv;
      const int n0 = act ? tile_of(u) * C::BN : 0;
      // a removed block of this pair (listed for another pair): P = 0
      const bool live = !BLK || !act || sblk[pr * bstride + n0 / kBlk - kb_base] != 0;
      f32x16 s[C::NB];
      // ---- M(u): S^T of tile u --------------------------------------------
      if (act && live) {
        const char* sK = smem + C::KOFF + (u % C::SLOTS) * C::TILEB;
#pragma unroll
        for (int bb = 0; bb < C::NB; ++bb) s[bb] = f32x16{};
#pragma unroll
        for (int kc = 0; kc < C::KC; ++kc)
#pragma unroll
          for (int bb = 0; bb < C::NB; ++bb)
            s[bb] = M::mma(as_v8<V8>(lds_read16(sK + bb * 32 * C::ROWB + koff[kc])), qf[kc], s[bb]);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < C::NB * C::KC - 4; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
#pragma unroll
        for (int bb = 0; bb < C::NB; ++bb) pin(s[bb]);
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // X(u)
      __builtin_amdgcn_sched_barrier(0);
      // ---- V(u): softmax of tile u -> exchange buffer u % NX ---------------
      if (act && !live) {
        char* x = xp(u);
#pragma unroll
        for (int i = 0; i < 2 * C::NB; ++i) *(V8*)(x + i * 1024 + lane * 16) = V8{};
        *(float*)(x + C::XP + lane * 4) = 1.f;
      } else if (act) {
        // element (bb, r) is key n0 + 32 bb + 8 (r / 4) + 4 h + r % 4
        if constexpr (!RAW) {
          const float fb = (float)(my_m - n0 - 4 * h);  // i - j = fb - (32 bb + 8 (r / 4) + r % 4)
#pragma unroll
          for (int bb = 0; bb < C::NB; ++bb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              float tv;
              s[bb][r] = score_log2_d<SOFTCAP, ALIBI>(s[bb][r], p, slope_log2,
                                                     fb - (float)(32 * bb + 8 * (r >> 2) + (r & 3)), tv);
            }
        }
        const int tn = n0 / C::BN;
        if (tn < tm_lo || tn >= tm_hi) {
          const int a0 = row_lo - n0 - 4 * h;
#pragma unroll
          for (int bb = 0; bb < C::NB; ++bb) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if ((unsigned)(32 * bb + 8 * (r >> 2) + (r & 3) - a0) >= row_w) s[bb][r] = kNegInf;
            pin(s[bb]);
          }
        }
        float mp[2 * C::NB];
#pragma unroll
        for (int bb = 0; bb < C::NB; ++bb) max16_partial(s[bb], mp[2 * bb], mp[2 * bb + 1]);
        float mx;
        if constexpr (C::NB == 1) mx = max2(mp[0], mp[1]);
        else mx = max2(max3(mp[0], mp[1], mp[2]), mp[3]);
        if constexpr (RAW) mx *= c2;
        mx = fmaxf(mx, swap_halves(mx));
        if (mx != mx) mx = kNegInf;
        const bool grow = mx > m_run + kWsRescaleThreshold;
        float alpha = 1.f;
        if (__builtin_amdgcn_ballot_w64(grow)) {
          const float m_new = grow ? mx : m_run;
          alpha = grow ? fast_exp2(m_run - m_new) : 1.f;
          l_run *= alpha;
          m_run = m_new;
        }
        const float m_use = (m_run == kNegInf) ? 0.f : m_run;
        char* x = xp(u);
        float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int bb = 0; bb < C::NB; ++bb) {
          f32x16 e;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            if constexpr (RAW) e[r] = fast_exp2(__builtin_fmaf(s[bb][r], c2, -m_use));
            else e[r] = fast_exp2(s[bb][r] - m_use);
            rs[r & 3] += e[r];
          }
          *(V8*)(x + (2 * bb) * 1024 + lane * 16) = pack8<T>(e, 0);
          *(V8*)(x + (2 * bb + 1) * 1024 + lane * 16) = pack8<T>(e, 8);
        }
        l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
        *(float*)(x + C::XP + lane * 4) = alpha;
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // Y(u)
      __builtin_amdgcn_sched_barrier(0);
    }
    // 1 / l to the partner, LSE out
    const float l_tot = l_run + swap_halves(l_run);
    const bool empty = !(l_tot > 0.f);
    *(float*)(xp(0) + C::XP + lane * 4) = empty ? 0.f : 1.0f / l_tot;
    if (my_m < p.Sq && h == 0)
      a.lse[(int64_t)(b * p.Hq + hq) * p.Sq + my_m] = empty ? kNegInf : (m_run + log2f(l_tot)) * kLn2;
    __syncthreads();  // E
  } else {
    // ================ PV-wave: tile copies, O^T += V^T P^T ==================
    const T* kp = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh;
    const T* vp = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh;
    const unsigned lds0 = lds_addr_of(smem);
    // Copy of tile v (walk index; past the end the last tile again) into
    // slot v % SLOTS of the K or V ring: E 1 KB loads, lane l of load e
    // covering physical chunk q of the tile (rows clamped to Skv - 1).
    int crow[C::E], kchk[C::E], vchk[C::E];
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int q = (pr * C::E + e) * 64 + lane;
      crow[e] = q / C::CPR;
      kchk[e] = swz_col<C::CPR>(crow[e], q % C::CPR);
      vchk[e] = swz_tr_inv<C::CPR>(crow[e], q % C::CPR);
    }
    auto copy = [&](const T* base, int64_t ss, const int (&chk)[C::E], int ring, int v) {
      const int n0 = tile_of(min(v, nv - 1)) * C::BN;
      const unsigned dst = lds0 + ring + (v % C::SLOTS) * C::TILEB + pr * C::E * 1024;
#pragma unroll
      for (int e = 0; e < C::E; ++e) {
        const int64_t n = min(n0 + crow[e], p.Skv - 1);
        load_lds16(base + n * ss + chk[e] * 8, dst + e * 1024);
      }
    };
    auto copy_k = [&](int v) { copy(kp, a.k.ss, kchk, C::KOFF, v); };
    auto copy_v = [&](int v) { copy(vp, a.v.ss, vchk, C::VOFF, v); };
    // transpose-read offsets (as fwd_mfma.hip)
    int voff[C::DB];
    {
      const int tr_row = 4 * h + ((lane & 15) >> 2);
      const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
        voff[db] = tr_row * C::ROWB + swz_tr<C::CPR>(tr_row, 4 * db + (tr_col >> 3)) * 16 + (tr_col & 7) * 2;
    }
    f32x16 acc[C::DB];
#pragma unroll
    for (int db = 0; db < C::DB; ++db) acc[db] = f32x16{};

    // Four slots: prologue K0 V0 K1 V1 K2, then K tile u+3 and V tile u+2 in
    // M(u).  At the end of V(u) K tile u+1 and V tile u have landed when at
    // most the 4E loads of M(u-1) and M(u) are in flight (for u = 0, 1 those
    // issued after K1 and after K2 in the prologue are 4E as well).
    // Two slots: prologue K0 K1, then V tile u in M(u) (into the slot of V
    // tile u-2, read in V(u-1)) and K tile u+2 in V(u) after the MFMAs (the
    // slot of K tile u, read in M(u)).  At the end of V(u) K tile u+1 and V
    // tile u have landed when at most the E loads of K tile u+2 are in flight.
    constexpr int WAITN = C::SLOTS == 4 ? 4 * C::E : C::E;
    if (nv > 0) {
      copy_k(0);
      if constexpr (C::SLOTS == 4) {
        copy_v(0);
        copy_k(1);
        copy_v(1);
        copy_k(2);
      } else {
        copy_k(1);
      }
      wait_vmcnt<WAITN>();  // K0 landed
    }
    __syncthreads();  // prologue
    for (int u = 0; u <= nv; ++u) {
      const bool act = u > 0;
      // ---- M(u): copies, P / alpha of tile u-1, first transpose reads -------
      if (nv > 0) {
        if constexpr (C::SLOTS == 4) {
          copy_k(u + 3);
          copy_v(u + 2);
        } else {
          copy_v(u);
        }
      }
      V8 P[2 * C::NB];
      float alpha = 1.f;
      i16x4 blo[C::RA + 1], bhi[C::RA + 1];
      const char* sV = smem + C::VOFF + ((u + C::SLOTS - 1) % C::SLOTS) * C::TILEB;  // V tile u-1
      // MFMA j: keys 16 (j / DB) .. + 15 of the tile, O^T rows 32 (j % DB) .. + 31
      auto rdV = [&](int j, i16x4& lo, i16x4& hi) {
        const char* vr = sV + 16 * (j / C::DB) * C::ROWB + voff[j % C::DB];
        lo = lds_read_tr4(vr);
        hi = lds_read_tr4(vr + 8 * C::ROWB);
      };
      if (act) {
        const char* x = xp(u - 1);
#pragma unroll
        for (int i = 0; i < 2 * C::NB; ++i) P[i] = *(const V8*)(x + i * 1024 + lane * 16);
        alpha = *(const float*)(x + C::XP + lane * 4);
#pragma unroll
        for (int j = 0; j < C::RA; ++j) rdV(j, blo[j], bhi[j]);
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // X(u)
      __builtin_amdgcn_sched_barrier(0);
      // ---- V(u): O^T of tile u-1 --------------------------------------------
      if (act) {
        if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
          for (int db = 0; db < C::DB; ++db) scale_inplace(acc[db], alpha);
        }
#pragma unroll
        for (int j = 0; j < 2 * C::NB * C::DB; ++j) {
          __builtin_amdgcn_sched_barrier(0);
          if (j + C::RA < 2 * C::NB * C::DB)
            rdV(j + C::RA, blo[(j + C::RA) % (C::RA + 1)], bhi[(j + C::RA) % (C::RA + 1)]);
          const V8 av = cat_tr<V8>(blo[j % (C::RA + 1)], bhi[j % (C::RA + 1)]);
          acc[j % C::DB] = M::mma(av, P[j / C::DB], acc[j % C::DB]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (C::SLOTS == 2) {
        if (nv > 0) copy_k(u + 2);
      }
      if (nv > 0) wait_vmcnt<WAITN>();  // K tile u+1, V tile u
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // Y(u)
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<0>();  // no copy may land after the workgroup's LDS is released
    __syncthreads();  // E: 1 / l is in the exchange buffer, every ring read is done
    const float inv = *(const float*)(xp(0) + C::XP + lane * 4);
    // O through the K ring (free now): this pair's 32 x D row-major tile,
    // 16-byte chunk c of row r at c ^ (r % CPR), then row-contiguous stores.
    char* so = smem + C::KOFF + pr * 32 * C::ROWB;
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 4 * db + i;  // columns 32 db + 8 i .. + 7; this lane's half at byte 8 h
        *(i32x2*)(so + l32 * C::ROWB + (c ^ (l32 % C::CPR)) * 16 + 8 * h) =
            pack4<T>(acc[db][4 * i] * inv, acc[db][4 * i + 1] * inv, acc[db][4 * i + 2] * inv,
                     acc[db][4 * i + 3] * inv);
      }
    }
    constexpr int RPI = 64 / C::CPR;  // rows per store instruction
    const int cc = lane % C::CPR;
    T* ob = (T*)a.o.data + b * a.o.sb + hq * a.o.sh + cc * 8;
#pragma unroll
    for (int k = 0; k < 32 / RPI; ++k) {
      const int rr = k * RPI + lane / C::CPR;
      const i32x4 x = lds_read16(so + rr * C::ROWB + (cc ^ (rr % C::CPR)) * 16);
      if (mw + rr < p.Sq) *(i32x4*)(ob + (int64_t)(mw + rr) * a.o.ss) = x;
    }
  }
}

// dynamic LDS of the block-sparse form: the pairs' block-map rows and the tile list
static size_t ws_dyn_lds(const Shape& p, int bstride) {
  return p.blk ? (size_t)WsCfg::NP * bstride + 2 * (size_t)((p.Skv + WsCfg::BN - 1) / WsCfg::BN + 2) : 0;
}
bool fwd_ws_fits(const Shape& p) {
  return WsCfg::LDSB + ws_dyn_lds(p, (p.blk_nk + 3) & ~3) <= 160 * 1024;
}

template <class T>
hipError_t launch_fwd_ws(const FwdArgs& a, hipStream_t st) {
  using C = WsCfg;
  FwdArgs x = a;
  const int gp = a.p.G & (-a.p.G);
  x.gpack = gp < C::NP ? gp : C::NP;
  const int bmh = 32 * (C::NP / x.gpack);
  x.nqt = (a.p.Sq + bmh - 1) / bmh;
  x.bstride = (a.p.blk_nk + 3) & ~3;
  const size_t dyn = ws_dyn_lds(a.p, x.bstride);
  const dim3 grid(x.nqt * (a.p.G / x.gpack) * a.p.B * a.p.Hkv), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  if (a.p.blk) {
    if (sc && al) hipLaunchKernelGGL((fwd_ws_kernel<T, true, true, true>), grid, block, dyn, st, x);
    else if (sc) hipLaunchKernelGGL((fwd_ws_kernel<T, true, false, true>), grid, block, dyn, st, x);
    else if (al) hipLaunchKernelGGL((fwd_ws_kernel<T, false, true, true>), grid, block, dyn, st, x);
    else hipLaunchKernelGGL((fwd_ws_kernel<T, false, false, true>), grid, block, dyn, st, x);
  } else {
    if (sc && al) hipLaunchKernelGGL((fwd_ws_kernel<T, true, true, false>), grid, block, 0, st, x);
    else if (sc) hipLaunchKernelGGL((fwd_ws_kernel<T, true, false, false>), grid, block, 0, st, x);
    else if (al) hipLaunchKernelGGL((fwd_ws_kernel<T, false, true, false>), grid, block, 0, st, x);
    else hipLaunchKernelGGL((fwd_ws_kernel<T, false, false, false>), grid, block, 0, st, x);
  }
  return hipGetLastError();
}

hipError_t fwd_ws_bf16_d256(const FwdArgs& a, hipStream_t st) { return launch_fwd_ws<__bf16>(a, st); }
hipError_t fwd_ws_f16_d256(const FwdArgs& a, hipStream_t st) { return launch_fwd_ws<_Float16>(a, st); }

#endif  // FLEXATT_D == 256

}  // namespace flexatt

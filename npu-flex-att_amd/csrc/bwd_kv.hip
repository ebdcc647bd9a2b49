// Flash-attention backward dK/dV for fp16/bf16 on gfx950 MFMA (KV-stationary
// tile stream, wave-specialised pairs).
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
//  * One workgroup = 128 KV rows of one (b, hkv) and 8 waves: four pairs, the
//    two waves of a pair on one SIMD (waves p and p + 4) and both owning the
//    same 32 KV rows (lane = KV row):
//      - the S-wave (p) holds the K and V rows as MFMA B operands, computes
//        S = Q K^T and dP = dO V^T, then P and dS on the VALU, and hands the
//        packed P / dS to its partner through LDS;
//      - the KV-wave (p + 4) holds dK^T / dV^T in registers, runs
//        dV^T += dO^T P and dK^T += Q^T dS, and issues all tile copies.
//    A single wave per SIMD cannot overlap its own VALU work with its MFMAs
//    (each MFMA blocks the issuing wave for a large part of its duration);
//    two waves per SIMD overlap the S-wave's VALU work with the KV-wave's
//    MFMAs.
//  * The workgroup walks one stream of tiles: for each of the G query heads of
//    the group, the 32-row query tiles that can attend to its KV rows.  A tile
//    is Q, dO (32 x D each), LSE and Delta (32 floats each), copied global ->
//    LDS with direct-to-LDS loads four tiles ahead into six stages.
//  * Step u has two phases separated by workgroup barriers:
//      M(u): S-wave: the 16 S / dP MFMAs of tile u, with the reads of its
//            LSE (converted to log2 units) and Delta (the dP MFMAs start
//            from Delta and run on -V, so they end at Delta - dP and
//            P (dP - Delta) is one multiply);  KV-wave: reads the packed
//            P / dS of tile u-1 and the first transpose reads;
//      V(u): S-wave: P / dS of tile u (VALU), written to the exchange buffer;
//            KV-wave: the 16 dV / dK MFMAs of tile u-1, the staged dS stores
//            of tile u-1 (when staged), then waits for tile u+1;
//    so that each SIMD alternates between the S-wave's MFMAs and the
//    KV-wave's MFMAs beside the S-wave's VALU work.  The KV-wave issues the
//    copies of tile u+4 in M(u): a global -> LDS copy holds its wave for
//    tens of cycles at issue, which the MFMA phases cannot afford.
//  * At D = 128 without block maps a step runs two consecutive tiles of the
//    walk (TPS = 2): 32 MFMAs per wave and phase, one exchange buffer of two
//    tiles, and the copies of the next step's two tiles in M(u).
//  * Q and dO are read two ways from the same tile, as rows (S, dP) and as
//    columns (dV^T, dK^T, with the LDS transpose read); the dual-use swizzle
//    keeps both conflict-free.
//  * Tiles that cross the causal diagonal, the window edge or the Q / KV
//    tails form P and dS with the per-element mask.
// Deterministic: every output element is owned by one lane and accumulated in
// a fixed order.
#include "flexatt_device.h"
#include "flexatt_kernels.h"

#ifndef FLEXATT_D
#error "FLEXATT_D (head dim) must be defined"
#endif

namespace flexatt {

#if FLEXATT_D == 128 || FLEXATT_D == 64 || FLEXATT_D == 256

template <int D, int TPS = 1>
struct KvCfg {
  static constexpr int NP = 4;                     // wave pairs, one per SIMD
  static constexpr int NW = 2 * NP;                // waves per workgroup
  static constexpr int BKV = 32 * NP;              // KV rows per workgroup
  static constexpr int BM = 32;                    // query rows per tile
  static constexpr int KC = D / 16;                // k chunks of the S / dP MFMAs
  static constexpr int DB = D / 32;                // 32-column blocks of dK / dV
  static constexpr int CPR = D / 8;                // 16-byte chunks per row
  static constexpr int ROWB = 2 * D;               // bytes per row
  static constexpr int TILEB = BM * ROWB;          // one of Q / dO
  static constexpr int E = TILEB / (1024 * NP);    // 1 KB copies per KV-wave per tensor
  static constexpr int STAGEB = 2 * TILEB + 2 * BM * 4;  // Q, dO, LSE, Delta
  // D = 64: five stages, so that two workgroups (74 KB of LDS each) share a
  // CU at four waves per SIMD; D = 128: six stages, one workgroup per CU;
  // D = 256: four (32 KB each)
  static constexpr int STAGES = D == 64 ? 5 : (D == 128 ? 6 : 4);
  static constexpr int WPE = D == 64 ? 4 : 2;      // waves per SIMD the register budget targets
  static constexpr int AHEAD = STAGES - 2;         // tile u + AHEAD is copied in step u
  // D = 256 runs dV and dK in two passes (the dV items and the dK items of one
  // launch, bwd_kv_passes_kernel), so that the KV-wave
  // holds one 128-register accumulator set; each pass exchanges one packed
  // operand (P, or dS) instead of both
  static constexpr bool PASSES = D == 256;
  static constexpr int XSLOTS = PASSES ? 2 : 4;    // 1 KB slots per pair: P, P, dS, dS (or P, P / dS, dS)
  static constexpr int XB = XSLOTS * 64 * 16;
  static constexpr int XOFF = STAGES * STAGEB;     // two exchange buffers (one of TPS tiles when TPS > 1)
  static constexpr int LDSB = XOFF + (TPS > 1 ? TPS : 2) * NP * XB;
  static constexpr int RPW = BM / NP;              // LSE / Delta rows copied per KV-wave
  static_assert(E * 1024 * NP == TILEB, "tile must split into 1 KB copies");
  static_assert(RPW == 8, "each KV-wave copies 8 LSE and 8 Delta values");
  static_assert(STAGEB % 256 == 0 && LDSB <= 160 * 1024, "LDS layout");
};

// PASS 0: dV and dK together; PASS 1: dV only; PASS 2: dK only (with the
// staged dS when DS).  TPS: tiles per step (two: both phases of a step run
// two consecutive tiles of the walk, 32 MFMAs per wave and phase, with one
// exchange buffer; D = 128 without block maps).
// The tile stream of one work item: KV block kb of (b, hkv) = bh, walked as
// workgroup slot `slot` (which sets the walk direction), in the LDS at smem.
template <class T, int D, bool SOFTCAP, bool ALIBI, bool DS, int PASS, bool BLK, int TPS = 1>
__device__ __forceinline__ void kv_tile_stream(const BwdArgs& a, char* smem, int slot, int kb, int bh) {
  using C = KvCfg<D, TPS>;
  static_assert(TPS == 1 || (TPS == 2 && PASS == 0 && !BLK && D == 128), "two tiles per step: D = 128, no block maps");
  static_assert(C::DB == 2 * C::KC / 4 && (D == 64 || D == 128 || D == 256), "head dims 64, 128, 256");
  static_assert((PASS == 0) != C::PASSES && !(DS && PASS == 1), "passes: D = 256 only; dS staged by the dK pass");
  constexpr bool DOV = PASS != 2, DOK = PASS != 1;  // accumulate dV / dK
  // S-wave MFMAs per tile: S (and, for dK, dP)
  constexpr int NM = DOK ? 2 * C::KC : C::KC;
  // S-wave: the LSE rows are read with MFMA LREAD of the phase and converted
  // to log2 units over its last four MFMAs
  constexpr int LREAD = NM >= 16 ? 8 : 0, LCONV = NM - 4;
  // exchange slots of P and dS
  constexpr int SLOT_P = 0, SLOT_DS = C::XSLOTS == 4 ? 2 : 0;
  // KV-wave: transpose reads RAK MFMAs ahead (three at D = 64 without the
  // soft-cap, where the 128-register budget is tightest for that wave;
  // measured faster there, slower with the soft-cap)
  constexpr int RAK = (D == 64 && !SOFTCAP) ? 3 : 4;
  using M = Mfma<T>;
  using V8 = typename M::v8;

  const Shape& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pr = wave & (C::NP - 1);  // pair: KV rows [32 pr, 32 pr + 32) of the block
  const bool s_wave = wave < C::NP;
  const int h = lane >> 5, l32 = lane & 31;
  const int nkb = a.ntiles;
  const int hk = bh % p.Hkv, b = bh / p.Hkv;
  const int n0 = kb * C::BKV;
  const int kw0 = n0 + 32 * pr;  // first KV row of this pair
  const int my_kv = kw0 + l32;   // KV row of this lane

  // Query rows that can attend to this block's KV rows.
  int q_lo = 0, q_hi = p.Sq;
  if (p.causal) q_lo = n0;  // q >= kv >= n0
  if (p.window > 0) q_hi = min(q_hi, n0 + C::BKV + p.window);  // q - kv <= W
  const int qt_lo = q_lo / C::BM;
  const int nqt = q_hi > q_lo ? (q_hi + C::BM - 1) / C::BM - qt_lo : 0;
  int ntile = p.G * nqt;
  // Tile order: the G heads of a query tile consecutively; the first round
  // of workgroups (one per CU) walks the query tiles from the last one down,
  // later ones (causal) from the diagonal up.  The first round starts
  // together at the last query tile; a later block of b blocks' length ends
  // when the first round's partner ends, so it starts b time units in and
  // reaches query tile 4 b + s at time b + s, the same tile for every later
  // block: in both rounds the KV blocks of one (b, hkv) read the Q / dO
  // stream in step and each tile is fetched from HBM about once.
  const int qt_top = qt_lo + nqt - 1;
  const bool up = p.causal && slot >= a.nstatic;
  const int qt0 = up ? qt_lo : qt_top, qt_end = up ? qt_top : qt_lo, qstep = up ? 1 : -1;

  // Block-sparse maps (BLK): the query tiles, in walk order, whose 128 x 128
  // block with this KV block is computed for some head of the group; the walk
  // visits only those (nlive of them), every head of each.  Heads whose own
  // block is removed in a listed tile skip their S-wave work (below).
  extern __shared__ unsigned short qlist[];
  __shared__ int s_nlive;
  int nlive = nqt;
  if constexpr (BLK) {
    if (wave == 0) {
      const int kbc = min(n0, p.Skv - 1) / kBlk;
      const int nh = p.blk_h > 1 ? p.G : 1;  // heads with a row of their own
      int base = 0;
      for (int i0 = 0; i0 < nqt; i0 += 64) {
        const int i = i0 + lane;
        bool live = false;
        if (i < nqt) {
          const int qt = qt0 + i * qstep;
          for (int g = 0; g < nh && !live; ++g)
            live = block_row(p, b, hk * p.G + g, min(qt * C::BM, p.Sq - 1))[kbc] != 0;
        }
        const unsigned long long m = __builtin_amdgcn_ballot_w64(live);
        if (live) qlist[base + __builtin_popcountll(m & ((1ull << lane) - 1))] = (unsigned short)(qt0 + i * qstep);
        base += __builtin_popcountll(m);
      }
      if (lane == 0) s_nlive = base;
    }
    __syncthreads();
    nlive = __builtin_amdgcn_readfirstlane(s_nlive);
  }
  // query tile of walk position i (BLK), the head of step u being u % G
  auto qt_at = [&](int i) -> int { return __builtin_amdgcn_readfirstlane((int)qlist[i]); };
  if constexpr (BLK) ntile = p.G * nlive;

  // Lane-constant LDS byte offsets of the row reads (S-wave) and the
  // transpose reads (KV-wave) within a tile.
  int rowoff[C::KC], voff_lo[C::DB], voff_hi[C::DB];
#pragma unroll
  for (int kc = 0; kc < C::KC; ++kc) rowoff[kc] = l32 * C::ROWB + swz_dual<C::CPR>(l32, 2 * kc + h) * 16;
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
  // This lane's 16-byte slot of packed operand i (SLOT_P, + 1: P; SLOT_DS,
  // + 1: dS) in the exchange buffer of tile u.
  auto xslot = [&](int u, int i) {
    return smem + C::XOFF + (u & 1) * (C::NP * C::XB) + pr * C::XB + i * 1024 + lane * 16;
  };

  if (s_wave) {
    // ======================= S-wave: S / dP MFMAs, P / dS ====================
    V8 kreg[C::KC], vreg[C::KC];  // K / V rows as B operands (k = 8 consecutive d)
    {
      const int r = min(my_kv, p.Skv - 1);
      const T* kr = (const T*)a.k.data + b * a.k.sb + hk * a.k.sh + (int64_t)r * a.k.ss + 8 * h;
      const T* vr = (const T*)a.v.data + b * a.v.sb + hk * a.v.sh + (int64_t)r * a.v.ss + 8 * h;
#pragma unroll
      for (int kc = 0; kc < C::KC; ++kc) {
        kreg[kc] = as_v8<V8>(ld_global16(kr + 16 * kc));
        // -V: the dP MFMAs start from Delta and so end at Delta - dP (below)
        if constexpr (DOK)
          vreg[kc] = as_v8<V8>(ld_global16(vr + 16 * kc) ^ i32x4{(int)0x80008000, (int)0x80008000,
                                                                  (int)0x80008000, (int)0x80008000});
      }
    }
    constexpr bool RAW = !SOFTCAP && !ALIBI;
    const float c2 = p.scale_log2;
    const bool kv_tail = kw0 + 32 > p.Skv;
    // Interval masks (document masks, PrefixLM): the query rows [clo, chi)
    // that may attend this lane's KV row; a tile needs no per-element test
    // when it lies inside [clo of the pair's last KV row, chi of its first)
    // (the bounds are non-decreasing).
    int clo, chi, pc_lo = 0, pc_hi = 0x7fffffff;
    col_bounds(p, b, min(my_kv, p.Skv - 1), clo, chi);
    if (p.docc) {
      int l0, h0, l1, h1;
      col_bounds(p, b, min(kw0, p.Skv - 1), l0, h0);
      col_bounds(p, b, min(kw0 + 31, p.Skv - 1), l1, h1);
      pc_lo = l1;
      pc_hi = h0;
    }
    // The query rows this lane's KV row may meet, as one interval
    // [q_lo, q_lo + q_w): causal, window, query tail, KV tail and column
    // bounds, so that a masked tile tests each element with one unsigned
    // compare against its offset.
    int q_lo = max(clo, 0), q_hi = min(chi, p.Sq);
    if (p.causal) q_lo = max(q_lo, my_kv);
    if (p.window > 0) q_hi = min(q_hi, my_kv + p.window + 1);
    if (my_kv >= p.Skv) q_hi = q_lo;
    const unsigned q_w = (unsigned)max(q_hi - q_lo, 0);
    int cg = 0, cqt = qt0;  // tile being formed (head, query tile)
    int sc = 0;               // its stage
    // Block-sparse maps: the byte of tile u's 128 x 128 block, loaded one
    // step ahead (the S-wave has no other memory operation in flight, so the
    // wait at its use is for this load alone).  A removed tile that is still
    // walked (a listed tile whose block is removed for this head, or a walk
    // without the list) skips the S-wave's MFMAs and VALU work: its P and dS
    // are written as zeros.
    auto blk_byte = [&](int g, int qt) -> int {
      return block_row(p, b, hk * p.G + g, min(qt * C::BM, p.Sq - 1))[min(kw0, p.Skv - 1) / kBlk];
    };
    int blk_next = 1;
    if (p.blk && ntile > 0) blk_next = blk_byte(0, BLK ? qt_at(0) : qt0);

    if constexpr (TPS > 1) {
      // Step u: tiles TPS u + w (w < TPS) of the walk, in stages sc + w.
      // Both tiles' 2 NM MFMAs run as one stream with one read-ahead ring;
      // past the end of the walk a tile's P and dS are written as zeros.
      const int nstep = (ntile + TPS - 1) / TPS;
      // This lane's 16 bytes of exchange slot i of tile w of the step.
      auto xs = [&](int w, int i) { return smem + C::XOFF + pr * (TPS * C::XB) + (w * C::XSLOTS + i) * 1024 + lane * 16; };
      __syncthreads();  // prologue: the first step's tiles landed
      for (int u = 0; u <= nstep; ++u) {
        f32x16 S[TPS], DP[TPS];
        f32x4 L4[TPS][4];
        if (u < nstep) {
          int ra[TPS][C::KC];
          const float* sR[TPS];
#pragma unroll
          for (int w = 0; w < TPS; ++w) {
            const int st = sc + w < C::STAGES ? sc + w : sc + w - C::STAGES;
#pragma unroll
            for (int kc = 0; kc < C::KC; ++kc) ra[w][kc] = rowoff[kc] + st * C::STAGEB;
            sR[w] = (const float*)(smem + st * C::STAGEB + 2 * C::TILEB);
            f32x4 D4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) D4[i] = __builtin_bit_cast(f32x4, lds_read16(sR[w] + 16 * i + 8 + 4 * h));
            DP[w] = f32x16{D4[0][0], D4[0][1], D4[0][2], D4[0][3], D4[1][0], D4[1][1], D4[1][2], D4[1][3],
                           D4[2][0], D4[2][1], D4[2][2], D4[2][3], D4[3][0], D4[3][1], D4[3][2], D4[3][3]};
            S[w] = f32x16{};
          }
          constexpr int NT = TPS * NM;
          // MFMA kk: tile kk / NM, its MFMA kk % NM (alternating the tiles' MFMAs measured slower)
          auto wk = [&](int kk, int& w, int& k) { w = kk / NM; k = kk % NM; };
          auto rdA = [&](int kk) {
            int w, k;
            wk(kk, w, k);
            return lds_read16(smem + (ra[w][k >> 1] + (k & 1) * C::TILEB));
          };
          // Q / dO rows read SAK MFMAs ahead (six: 0.5% faster than four over
          // the 64 MFMAs of a two-tile step; eight is slower)
          constexpr int SAK = 6;
          i32x4 ab[SAK + 1];
#pragma unroll
          for (int kk = 0; kk < SAK; ++kk) ab[kk] = rdA(kk);
#pragma unroll
          for (int kk = 0; kk < NT; ++kk) {
            __builtin_amdgcn_sched_barrier(0);
            if (kk + SAK < NT) ab[(kk + SAK) % (SAK + 1)] = rdA(kk + SAK);
            int w, k;
            wk(kk, w, k);
            if (k == LREAD) {
#pragma unroll
              for (int i = 0; i < 4; ++i) L4[w][i] = __builtin_bit_cast(f32x4, lds_read16(sR[w] + 16 * i + 4 * h));
            }
            if (k >= LCONV) {
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) L4[w][k - LCONV][jj] *= kLog2e;
            }
            if (k & 1) DP[w] = M::mma(as_v8<V8>(ab[kk % (SAK + 1)]), vreg[k >> 1], DP[w]);
            else S[w] = M::mma(as_v8<V8>(ab[kk % (SAK + 1)]), kreg[k >> 1], S[w]);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int w = 0; w < TPS; ++w) {
            pin(S[w]);
            pin(DP[w]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // X(u)
        __builtin_amdgcn_sched_barrier(0);
        if (u < nstep) {
#pragma unroll
          for (int w = 0; w < TPS; ++w) {
            if (TPS * u + w >= ntile) {
#pragma unroll
              for (int i = 0; i < C::XSLOTS; ++i) *(V8*)xs(w, i) = V8{};
              continue;
            }
            const int hq = hk * p.G + cg;
            const int m0 = cqt * C::BM;
            const float sl = ALIBI ? p.alibi[hq] * kLog2e : 0.f;
            if (++cg == p.G) {
              cg = 0;
              cqt += qstep;
            }
            // as the one-tile form below: element r is query row
            // m0 + 8(r/4) + 4h + r%4, KV row my_kv
            auto form = [&](auto masked) {
              f32x16 pe, de;
              float y[16], tt[16];
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                tt[r] = 0.f;
                if constexpr (RAW) {
                  y[r] = __builtin_fmaf(S[w][r], c2, -L4[w][r >> 2][r & 3]);
                } else {
                  const int q = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
                  y[r] = score_log2<SOFTCAP, ALIBI>(S[w][r], p, sl, q, my_kv, tt[r]) - L4[w][r >> 2][r & 3];
                }
              }
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                float e = fast_exp2(y[r]);
                if constexpr (decltype(masked)::value) {
                  const int a0 = q_lo - m0 - 4 * h;
                  e = (unsigned)(8 * (r >> 2) + (r & 3) - a0) < q_w ? e : 0.f;
                }
                pe[r] = e;
              }
              __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                float ds = -pe[r] * DP[w][r];
                if constexpr (SOFTCAP) ds *= 1.f - tt[r] * tt[r];
                de[r] = ds;
              }
              __builtin_amdgcn_sched_barrier(0);
              *(V8*)xs(w, SLOT_P) = pack8<T>(pe, 0);
              *(V8*)xs(w, SLOT_P + 1) = pack8<T>(pe, 8);
              *(V8*)xs(w, SLOT_DS) = pack8<T>(de, 0);
              *(V8*)xs(w, SLOT_DS + 1) = pack8<T>(de, 8);
            };
            if ((m0 + C::BM > p.Sq) || kv_tail || (p.causal && m0 < kw0 + 31) ||
                (p.window > 0 && m0 + C::BM - 1 - kw0 > p.window) || m0 < pc_lo || m0 + C::BM > pc_hi) {
              form(std::true_type{});
            } else {
              form(std::false_type{});
            }
          }
          sc += TPS;
          if (sc >= C::STAGES) sc -= C::STAGES;
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // Y(u)
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
    __syncthreads();  // prologue: tile 0 landed
    for (int u = 0; u <= ntile; ++u) {
      const bool act = u < ntile;
      f32x16 S, DP;        // Q K^T and Delta - dO V^T (the latter accumulated from Delta)
      f32x4 L4[4];         // LSE (to log2 units) of this lane's query rows
      bool live = true;
      if (p.blk && act) {
        live = __builtin_amdgcn_readfirstlane(blk_next) != 0;
        int ng, nq;
        if constexpr (BLK) {
          ng = (u + 1) % p.G;
          nq = u + 1 < ntile ? qt_at((u + 1) / p.G) : 0;
        } else {
          ng = cg + 1 == p.G ? 0 : cg + 1;
          nq = cg + 1 == p.G ? cqt + qstep : cqt;
        }
        if (u + 1 < ntile) blk_next = blk_byte(ng, nq);
      }
      // ---- M(u): S = Q K^T, DP = Delta - dO V^T of tile u; LSE reads ------
      if (act && live) {
        // Row-read addresses of this stage (the Q / dO choice folds into the
        // instruction offset).
        int ra[C::KC];
#pragma unroll
        for (int kc = 0; kc < C::KC; ++kc) ra[kc] = rowoff[kc] + sc * C::STAGEB;
        // MFMA k reads Q row chunk k (S only) or, interleaving S and dP,
        // chunk k / 2 of Q (even k) or dO (odd k)
        auto rdA = [&](int k) {
          if constexpr (DOK) return lds_read16(smem + (ra[k >> 1] + (k & 1) * C::TILEB));
          else return lds_read16(smem + ra[k]);
        };
        const float* sR = (const float*)(smem + sc * C::STAGEB + 2 * C::TILEB);
        i32x4 ab[5];
        S = f32x16{};
        if constexpr (DOK) {
          // Delta of the query rows m0 + 8i + 4h + j is the initial dP
          // accumulator (element 4i + j), so that P (dP - Delta) needs no
          // subtraction on the VALU.
          f32x4 D4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) D4[i] = __builtin_bit_cast(f32x4, lds_read16(sR + 16 * i + 8 + 4 * h));
          DP = f32x16{D4[0][0], D4[0][1], D4[0][2], D4[0][3], D4[1][0], D4[1][1], D4[1][2], D4[1][3],
                      D4[2][0], D4[2][1], D4[2][2], D4[2][3], D4[3][0], D4[3][1], D4[3][2], D4[3][3]};
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) ab[k] = rdA(k);
#pragma unroll
        for (int k = 0; k < NM; ++k) {
          __builtin_amdgcn_sched_barrier(0);
          if (k + 4 < NM) ab[(k + 4) % 5] = rdA(k + 4);
          if (k == LREAD) {  // query rows m0 + 8i + 4h + j
#pragma unroll
            for (int i = 0; i < 4; ++i) L4[i] = __builtin_bit_cast(f32x4, lds_read16(sR + 16 * i + 4 * h));
          }
          if (k >= LCONV) {  // LSE -> log2 units
            const int i = k - LCONV;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) L4[i][jj] *= kLog2e;
          }
          if constexpr (!DOK) S = M::mma(as_v8<V8>(ab[k % 5]), kreg[k], S);
          else if (k & 1) DP = M::mma(as_v8<V8>(ab[k % 5]), vreg[k >> 1], DP);
          else S = M::mma(as_v8<V8>(ab[k % 5]), kreg[k >> 1], S);
        }
        __builtin_amdgcn_sched_barrier(0);
        pin(S);
        if constexpr (DOK) pin(DP);
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // X(u)
      __builtin_amdgcn_sched_barrier(0);
      // ---- V(u): P, dS of tile u -> exchange buffer u & 1 -----------------
      if (act) {
        if constexpr (BLK) {  // tile u of the list walk
          cg = u % p.G;
          cqt = qt_at(u / p.G);
        }
        const int hq = hk * p.G + cg;
        const int m0 = cqt * C::BM;
        const float sl = ALIBI ? p.alibi[hq] * kLog2e : 0.f;
        if (++cg == p.G) {
          cg = 0;
          cqt += qstep;
        }
        sc = sc + 1 == C::STAGES ? 0 : sc + 1;
        // Element r is query row m0 + 8(r/4) + 4h + r%4, KV row my_kv.  Each
        // step runs over all 16 elements before the next one starts, so that
        // no instruction waits on the one just before it.
        auto form = [&](auto masked) {
          f32x16 pe, de;
          float y[16], tt[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            tt[r] = 0.f;
            if constexpr (RAW) {
              y[r] = __builtin_fmaf(S[r], c2, -L4[r >> 2][r & 3]);
            } else {
              const int q = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
              y[r] = score_log2<SOFTCAP, ALIBI>(S[r], p, sl, q, my_kv, tt[r]) - L4[r >> 2][r & 3];
            }
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float e = fast_exp2(y[r]);
            if constexpr (decltype(masked)::value) {
              const int a0 = q_lo - m0 - 4 * h;  // element offset of the interval's start
              e = (unsigned)(8 * (r >> 2) + (r & 3) - a0) < q_w ? e : 0.f;
            }
            pe[r] = e;
          }
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (DOK) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              float ds = -pe[r] * DP[r];  // P (dP - Delta)
              if constexpr (SOFTCAP) ds *= 1.f - tt[r] * tt[r];
              de[r] = ds;
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (DOV) {
            *(V8*)xslot(u, SLOT_P) = pack8<T>(pe, 0);
            *(V8*)xslot(u, SLOT_P + 1) = pack8<T>(pe, 8);
          }
          if constexpr (DOK) {
            *(V8*)xslot(u, SLOT_DS) = pack8<T>(de, 0);
            *(V8*)xslot(u, SLOT_DS + 1) = pack8<T>(de, 8);
          }
        };
        if (!live) {
          if constexpr (DOV) {
            *(V8*)xslot(u, SLOT_P) = V8{};
            *(V8*)xslot(u, SLOT_P + 1) = V8{};
          }
          if constexpr (DOK) {
            *(V8*)xslot(u, SLOT_DS) = V8{};
            *(V8*)xslot(u, SLOT_DS + 1) = V8{};
          }
        } else if ((m0 + C::BM > p.Sq) || kv_tail || (p.causal && m0 < kw0 + 31) ||
                   (p.window > 0 && m0 + C::BM - 1 - kw0 > p.window) || m0 < pc_lo || m0 + C::BM > pc_hi) {
          form(std::true_type{});
        } else {
          form(std::false_type{});
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // Y(u)
      __builtin_amdgcn_sched_barrier(0);
    }
    }  // TPS == 1
  } else {
    // ===================== KV-wave: copies, dV / dK MFMAs ====================
    f32x16 dk[C::DB], dv[C::DB];
#pragma unroll
    for (int db = 0; db < C::DB; ++db) {
      dk[db] = f32x16{};
      dv[db] = f32x16{};
    }
    // Tile copies: tile t -> stage t % STAGES; past the end, redundant copies
    // of the last tile into a free stage keep every KV-wave at 2E + 1 copy
    // operations per tile.
    const unsigned lds0 = lds_addr_of(smem);
    int crow[C::E], cchk[C::E];  // row / logical chunk of this lane in copy e
#pragma unroll
    for (int e = 0; e < C::E; ++e) {
      const int q = (pr * C::E + e) * 64 + lane;
      crow[e] = q / C::CPR;
      cchk[e] = swz_dual_inv<C::CPR>(crow[e], q % C::CPR);
    }
    // Per tile only scalar bases move; the per-lane offsets are recomputed
    // (clamped to row Sq - 1) only for a query-tail tile.
    const int rl = C::RPW * pr + (lane & 7);  // LSE / Delta row of this lane's copy
    int64_t cq[C::E], co[C::E];
    int crl;
    auto set_offsets = [&](int last) {  // last = Sq - 1 - m0 (clamp)
#pragma unroll
      for (int e = 0; e < C::E; ++e) {
        const int64_t r = min(crow[e], last);
        cq[e] = (r * a.q.ss + cchk[e] * 8) * (int64_t)sizeof(T);
        co[e] = (r * a.dout.ss + cchk[e] * 8) * (int64_t)sizeof(T);
      }
      crl = min(rl, last);
    };
    // Byte steps: to the next head of the group, and from the last head of a
    // query tile back to the first head of the next query tile.
    const int64_t qh = a.q.sh * (int64_t)sizeof(T), oh = a.dout.sh * (int64_t)sizeof(T);
    const int64_t qwrap = (int64_t)qstep * C::BM * a.q.ss * (int64_t)sizeof(T) - (int64_t)(p.G - 1) * qh;
    const int64_t owrap = (int64_t)qstep * C::BM * a.dout.ss * (int64_t)sizeof(T) - (int64_t)(p.G - 1) * oh;
    const int64_t lwrap = (int64_t)qstep * C::BM - (int64_t)(p.G - 1) * p.Sq;
    int is_g = 0, is_qt = qt0;  // next tile to copy (head, query tile)
    if constexpr (BLK) is_qt = nlive > 0 ? qt_at(0) : qt0;
    const char *qcur, *ocur;
    const float* lcur;  // LSE (lanes 0-7) or Delta (lanes 8-15) row m0
    auto point = [&](int g, int qt) {
      const int hq = hk * p.G + g;
      const int64_t m0 = (int64_t)qt * C::BM;
      qcur = (const char*)((const T*)a.q.data + b * a.q.sb + hq * a.q.sh + m0 * a.q.ss);
      ocur = (const char*)((const T*)a.dout.data + b * a.dout.sb + hq * a.dout.sh + m0 * a.dout.ss);
      lcur = (lane < 8 ? a.lse : a.delta) + (int64_t)(b * p.Hq + hq) * p.Sq + m0;
    };
    point(0, is_qt);
    int cu = 0;  // BLK: walk step of the next copy
    bool tail = false;
    auto prep = [&]() {  // per-lane offsets for the query tile is_qt
      const int m0 = is_qt * C::BM;
      const bool t = m0 + C::BM > p.Sq;
      if (t || tail) set_offsets(t ? p.Sq - 1 - m0 : C::BM);
      tail = t;
    };
    set_offsets(C::BM);
    prep();
    // Copy operation j (0 .. 2E) of the next tile, going to stage st.
    auto copy_op = [&](int st, int j) {
      const unsigned sb = lds0 + st * C::STAGEB;
      if (j < C::E) {
        load_lds16(qcur + cq[j], sb + (pr * C::E + j) * 1024);
      } else if (j < 2 * C::E) {
        load_lds16(ocur + co[j - C::E], sb + C::TILEB + (pr * C::E + j - C::E) * 1024);
      } else if (lane < 16) {
        load_lds4(lcur + crl, sb + 2 * C::TILEB + 64 * pr);
      }
    };
    auto advance = [&]() {  // past the end the last tile is copied again
      if constexpr (BLK) {
        if (cu + 1 < ntile) {
          ++cu;
          const int qt = qt_at(cu / p.G);
          is_g = cu % p.G;
          point(is_g, qt);
          if (qt != is_qt) {
            is_qt = qt;
            prep();
          }
        }
      } else if (is_g < p.G - 1 || is_qt != qt_end) {
        if (++is_g == p.G) {
          is_g = 0;
          is_qt += qstep;
          qcur += qwrap;
          ocur += owrap;
          lcur += lwrap;
          prep();
        } else {
          qcur += qh;
          ocur += oh;
          lcur += p.Sq;
        }
      }
    };
    constexpr int CNT = 2 * C::E + 1;  // copy operations per tile per KV-wave
    // Transpose reads (A operands of dV^T / dK^T) of MFMA j; tb_lo / tb_hi
    // are the lane addresses in the tile's stage (Q / dO and the 16-row block
    // fold into the instruction offset).
    int tb_lo[C::DB], tb_hi[C::DB];
    // MFMA j: d-block db, query half qc, dK (Q^T, dS) or dV (dO^T, P); both
    // interleaved (PASS 0) or one of them
    constexpr int NJ = (PASS == 0 ? 4 : 2) * C::DB;
    auto jmap = [&](int j, int& db, int& qc, bool& isk) {
      if constexpr (PASS == 0) {
        db = (j >> 1) % C::DB;
        qc = (j >> 1) / C::DB;
        isk = j & 1;
      } else {
        db = j % C::DB;
        qc = j / C::DB;
        isk = PASS == 2;
      }
    };
    auto rdB = [&](int j, i16x4& lo, i16x4& hi) {
      int db, qc;
      bool isk;
      jmap(j, db, qc, isk);
      const int off = (isk ? 0 : C::TILEB) + 16 * qc * C::ROWB;
      lo = lds_read_tr4(smem + (tb_lo[db] + off));
      hi = lds_read_tr4(smem + (tb_hi[db] + off));
    };
    int s_tr = 0, s_cp = C::AHEAD % C::STAGES;  // stages of tiles u-1 and u+AHEAD
    // Staged dS: tile u-1 (head ds_g, query tile ds_qt) leaves the exchange
    // buffer transposed, lane = query row, as two 1 KB fragments of this
    // pair's 32 KV rows (the dQ kernel's B operands).  Lane-constant part of
    // the transpose-read address: this lane (group g = lane / 16) gathers
    // query rows 4a .. 4a + 3, a = 4 (g & 1) + lane % 4, of KV row
    // 4 (lane / 32) + (lane % 16) / 4 (+ 16 f + 8 half), from where the
    // S-wave packed them (operand 2 + a / 4, lane (a & 1) * 32 + KV row,
    // byte 8 ((a / 2) & 1)).
    // dsp: this lane's 16 bytes of the unit of (head hk G + ds_g, query tile
    // ds_qt, this KV block), moved per tile with the band counts of the query
    // tiles it passes.
    int ds_g = 0, ds_qt = qt0;
    if constexpr (BLK) ds_qt = nlive > 0 ? qt_at(0) : qt0;
    int xtr = 0;
    char* dsp = nullptr;
    // this lane's 16 bytes of the unit of (head hk G + g, query tile qt, this KV block)
    auto ds_at = [&](int g, int qt) {
      const int64_t unit = (int64_t)(b * p.Hq + hk * p.G + g) * a.ds_head +
                           ds_tile_offset(qt, p.causal, p.window, nkb) + kb - ds_kb_lo(qt, p.window, nkb);
      return a.ds + unit * kDsUnitB + (2 * pr) * 1024 + lane * 16;
    };
    int su = 0;  // BLK: walk step of the next dS store
    if constexpr (DS) {
      const int aq = 4 * ((lane >> 4) & 1) + (lane & 3);
      const int jr = 4 * (lane >> 5) + ((lane & 15) >> 2);
      xtr = C::XOFF + pr * C::XB + (SLOT_DS + (aq >> 2)) * 1024 + (((aq & 1) << 5) + jr) * 16 + 8 * ((aq >> 1) & 1);
      dsp = ds_at(0, ds_qt);
    }

    if (TPS == 1 && ntile > 0) {
#pragma unroll
      for (int t = 0; t < C::AHEAD; ++t) {
#pragma unroll
        for (int j = 0; j < CNT; ++j) copy_op(t, j);
        advance();
      }
      wait_vmcnt<(C::AHEAD - 1) * CNT>();
    }
    // Staged dS of tile u-1 (st4, read from the exchange buffer in M(u)) to
    // its unit, and the unit cursor to the next tile.  Issued in V(u) after the
    // MFMAs at D = 128 and 256, where the KV-wave waits for the S-wave's VALU
    // work anyway (3% faster there), in M(u) at D = 64 (3% faster there); the
    // tile waits count the stores either way, as they precede them.
    constexpr bool DS_LATE = D != 64;
    // fragment f of the staged dS, streamed past the caches: each fragment
    // is read once, by the dQ kernel
    auto store_frag = [&](const i16x4 (&st4)[4], int f) {
      __builtin_nontemporal_store(__builtin_bit_cast(i32x4, cat_tr<V8>(st4[2 * f], st4[2 * f + 1])),
                                  (i32x4*)(dsp + f * 1024));
    };
    auto ds_next = [&]() {  // the unit cursor to the next tile
      if constexpr (BLK) {
        if (++su < ntile) dsp = ds_at(su % p.G, qt_at(su / p.G));
        return;
      }
      int64_t step;  // in units
      if (++ds_g == p.G) {
        // first head of the next query tile t: the unit index moves by
        // (offset(t) - kb_lo(t)) - (offset(t') - kb_lo(t')) from tile
        // t' = ds_qt, and offset(x + 1) - offset(x) = kb_hi(x) - kb_lo(x)
        const int t = ds_qt + qstep;
        step = (up ? ds_kb_hi(ds_qt, p.causal, nkb) - ds_kb_lo(t, p.window, nkb)
                   : ds_kb_lo(ds_qt, p.window, nkb) - ds_kb_hi(t, p.causal, nkb)) -
               (int64_t)(p.G - 1) * a.ds_head;
        ds_g = 0;
        ds_qt = t;
      } else {
        step = a.ds_head;
      }
      dsp += step * kDsUnitB;
    };
    auto store_ds = [&](const i16x4 (&st4)[4]) {
      store_frag(st4, 0);
      store_frag(st4, 1);
      ds_next();
    };
    if constexpr (TPS > 1) {
      // Step u: the dV / dK MFMAs of step u-1's tiles (TPS (u-1) + w, in
      // stages s_tr2 + w) in V(u); the copies of step u+1's tiles in M(u),
      // into the stages of step u-2's tiles (read in V(u-1)); so each copy
      // has one step to land.  The staged dS of step u-1's live tiles leaves
      // between the MFMAs, and the wait at the end of V(u) lets only those
      // stores stay in flight.
      const int nstep = (ntile + TPS - 1) / TPS;
      int s_cp2 = 0;  // stage of the next tile to copy
      auto copy_tile = [&]() {
#pragma unroll
        for (int j = 0; j < CNT; ++j) copy_op(s_cp2, j);
        advance();
        s_cp2 = s_cp2 + 1 == C::STAGES ? 0 : s_cp2 + 1;
      };
      if (ntile > 0) {
#pragma unroll
        for (int w = 0; w < TPS; ++w) copy_tile();
        wait_vmcnt<0>();
      }
      const int xtr2 = xtr + pr * (TPS - 1) * C::XB;  // staged-dS transpose reads: pair stride TPS XB
      auto xs = [&](int w, int i) { return smem + C::XOFF + pr * (TPS * C::XB) + (w * C::XSLOTS + i) * 1024 + lane * 16; };
      int s_tr2 = 0;  // stage of the first tile of step u-1
      __syncthreads();  // prologue
      for (int u = 0; u <= nstep; ++u) {
        const bool act = u > 0;
        const int na = act ? min(TPS, ntile - TPS * (u - 1)) : 0;  // tiles of step u-1 in the walk
        if (ntile > 0) {
#pragma unroll
          for (int w = 0; w < TPS; ++w) copy_tile();
        }
        V8 PP[TPS][2], PS[TPS][2];
        i16x4 blo[RAK + 1], bhi[RAK + 1];
        i16x4 st4[TPS][4];
        auto rdB2 = [&](int jj, i16x4& lo, i16x4& hi) {
          const int w = jj / NJ;
          int db, qc;
          bool isk;
          jmap(jj % NJ, db, qc, isk);
          const int st = s_tr2 + w < C::STAGES ? s_tr2 + w : s_tr2 + w - C::STAGES;
          const int off = (isk ? 0 : C::TILEB) + 16 * qc * C::ROWB + st * C::STAGEB;
          lo = lds_read_tr4(smem + (voff_lo[db] + off));
          hi = lds_read_tr4(smem + (voff_hi[db] + off));
        };
        if (act) {
#pragma unroll
          for (int w = 0; w < TPS; ++w) {
            PP[w][0] = *(const V8*)xs(w, SLOT_P);
            PP[w][1] = *(const V8*)xs(w, SLOT_P + 1);
            PS[w][0] = *(const V8*)xs(w, SLOT_DS);
            PS[w][1] = *(const V8*)xs(w, SLOT_DS + 1);
            if constexpr (DS) {
              const char* xb = smem + xtr2 + w * C::XSLOTS * 1024;
#pragma unroll
              for (int f = 0; f < 2; ++f) {
                st4[w][2 * f] = lds_read_tr4(xb + (16 * f) * 16);
                st4[w][2 * f + 1] = lds_read_tr4(xb + (16 * f + 8) * 16);
              }
            }
          }
#pragma unroll
          for (int jj = 0; jj < RAK; ++jj) rdB2(jj, blo[jj], bhi[jj]);
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // X(u)
        __builtin_amdgcn_sched_barrier(0);
        if (act) {
#pragma unroll
          for (int jj = 0; jj < TPS * NJ; ++jj) {
            __builtin_amdgcn_sched_barrier(0);
            if (jj + RAK < TPS * NJ) rdB2(jj + RAK, blo[(jj + RAK) % (RAK + 1)], bhi[(jj + RAK) % (RAK + 1)]);
            const int w = jj / NJ;
            int db, qc;
            bool isk;
            jmap(jj % NJ, db, qc, isk);
            const V8 av = cat_tr<V8>(blo[jj % (RAK + 1)], bhi[jj % (RAK + 1)]);
            if (isk) dk[db] = M::mma(av, PS[w][qc], dk[db]);
            else dv[db] = M::mma(av, PP[w][qc], dv[db]);
            if constexpr (DS) {
              // fragment f of tile t leaves after MFMA 3 + 8 (2 t + f): the
              // KV-waves' stores spread over the phase instead of meeting
              // at its end (1% faster than all four after the MFMAs; other
              // spacings measured slower)
              static_assert(TPS * NJ == 32, "four stores over 32 MFMAs");
              if (jj % 8 == 3) {
                const int t = jj >> 4, f = (jj >> 3) & 1;
                if (t < na) {
                  store_frag(st4[t], f);
                  if (f == 1) ds_next();
                }
              }
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          s_tr2 += TPS;
          if (s_tr2 >= C::STAGES) s_tr2 -= C::STAGES;
        }
        if (ntile > 0) {  // step u+1's tiles landed; this step's 2 na dS stores may stay in flight
          if (DS && na == 2) wait_vmcnt<4>();
          else if (DS && na == 1) wait_vmcnt<2>();
          else wait_vmcnt<0>();
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // Y(u)
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
    __syncthreads();  // prologue
    for (int u = 0; u <= ntile; ++u) {
      const bool act = u > 0;
      // ---- M(u): copies of tile u + AHEAD (a global -> LDS copy holds its
      //      wave for tens of cycles at issue, so they stay out of the MFMA
      //      phase), packed P / dS of tile u-1, first transpose reads --------
      V8 PP[2], PS[2];
      i16x4 blo[RAK + 1], bhi[RAK + 1];
      i16x4 st4[4];  // staged dS of tile u-1: read in M(u), stored in V(u)
      if (ntile > 0) {
#pragma unroll
        for (int j = 0; j < CNT; ++j) copy_op(s_cp, j);
      }
      if (act) {
#pragma unroll
        for (int db = 0; db < C::DB; ++db) {
          tb_lo[db] = voff_lo[db] + s_tr * C::STAGEB;
          tb_hi[db] = voff_hi[db] + s_tr * C::STAGEB;
        }
        if constexpr (DOV) {
          PP[0] = *(const V8*)xslot(u - 1, SLOT_P);
          PP[1] = *(const V8*)xslot(u - 1, SLOT_P + 1);
        }
        if constexpr (DOK) {
          PS[0] = *(const V8*)xslot(u - 1, SLOT_DS);
          PS[1] = *(const V8*)xslot(u - 1, SLOT_DS + 1);
        }
        if constexpr (DS) {
          const char* xb = smem + xtr + ((u - 1) & 1) * (C::NP * C::XB);
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            st4[2 * f] = lds_read_tr4(xb + (16 * f) * 16);
            st4[2 * f + 1] = lds_read_tr4(xb + (16 * f + 8) * 16);
          }
        }
#pragma unroll
        for (int j = 0; j < RAK; ++j) rdB(j, blo[j], bhi[j]);
        if constexpr (DS && !DS_LATE) store_ds(st4);
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // X(u)
      __builtin_amdgcn_sched_barrier(0);
      // ---- V(u): dV / dK of tile u-1 ---------------------------------------
      if (act) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          __builtin_amdgcn_sched_barrier(0);
          if (j + RAK < NJ) rdB(j + RAK, blo[(j + RAK) % (RAK + 1)], bhi[(j + RAK) % (RAK + 1)]);
          int db, qc;
          bool isk;
          jmap(j, db, qc, isk);
          const V8 av = cat_tr<V8>(blo[j % (RAK + 1)], bhi[j % (RAK + 1)]);
          if (isk) dk[db] = M::mma(av, PS[qc], dk[db]);
          else dv[db] = M::mma(av, PP[qc], dv[db]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (DS && DS_LATE) store_ds(st4);
        s_tr = s_tr + 1 == C::STAGES ? 0 : s_tr + 1;
      }
      if (ntile > 0) {
        advance();
        // tile u+1 landed.  Stores count in vmcnt too: with staged dS, the
        // two stores of each step s >= 1 from step u + 1 - AHEAD on
        // (2 min(u, AHEAD) of them) were issued after tile u+1's copies and
        // may stay in flight.
        if constexpr (DS) {
          static_assert(C::AHEAD <= 4, "wait counts below cover AHEAD <= 4");
          if (u >= C::AHEAD) wait_vmcnt<(C::AHEAD - 1) * CNT + 2 * C::AHEAD>();
          else if (u == 3) wait_vmcnt<(C::AHEAD - 1) * CNT + 6>();
          else if (u == 2) wait_vmcnt<(C::AHEAD - 1) * CNT + 4>();
          else if (u == 1) wait_vmcnt<(C::AHEAD - 1) * CNT + 2>();
          else wait_vmcnt<(C::AHEAD - 1) * CNT>();
        } else {
          wait_vmcnt<(C::AHEAD - 1) * CNT>();
        }
        s_cp = s_cp + 1 == C::STAGES ? 0 : s_cp + 1;
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // Y(u)
      __builtin_amdgcn_sched_barrier(0);
    }
    }  // TPS == 1
    wait_vmcnt<0>();  // redundant copies in flight must land before the workgroup ends

    // dK = scale * sum dS^T Q, dV = sum P^T dO; lane = KV row.
    if (my_kv < p.Skv) {
      T* kq = (T*)a.dk.data + b * a.dk.sb + hk * a.dk.sh + (int64_t)my_kv * a.dk.ss + 4 * h;
      T* vq = (T*)a.dv.data + b * a.dv.sb + hk * a.dv.sh + (int64_t)my_kv * a.dv.ss + 4 * h;
      const float sc = p.scale;
#pragma unroll
      for (int db = 0; db < C::DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (DOK)
            st_global8(kq + 32 * db + 8 * i, pack4<T>(dk[db][4 * i] * sc, dk[db][4 * i + 1] * sc,
                                                     dk[db][4 * i + 2] * sc, dk[db][4 * i + 3] * sc));
          if constexpr (DOV)
            st_global8(vq + 32 * db + 8 * i, pack4<T>(dv[db][4 * i], dv[db][4 * i + 1], dv[db][4 * i + 2],
                                                     dv[db][4 * i + 3]));
        }
    }
  }
}

// D = 64 and 128 (PASS 0).  Work item: (b, hkv, KV block), blocks of
// one (b, hkv) consecutive so that they share an XCD (and its L2) and heavy /
// light causal blocks interleave; block 0 has the longest causal band.
template <class T, int D, bool SOFTCAP, bool ALIBI, bool DS, int PASS, bool BLK, int TPS = 1>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(KvCfg<D>::WPE, KvCfg<D>::WPE)))
void bwd_kv_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) char smem[KvCfg<D, TPS>::LDSB];
  const int nkb = a.ntiles;
  const int slot = queue_slot(a.queue, a.nstatic);
  if (slot >= (int)gridDim.x) return;  // (a counter that was not cleared)
  int kb, bh;
  if (!xcd_lpt_item(slot, nkb, a.p.B * a.p.Hkv, kb, bh)) {
    const int w = xcd_remap(slot, gridDim.x);
    kb = w % nkb;
    bh = w / nkb;
  }
  kv_tile_stream<T, D, SOFTCAP, ALIBI, DS, PASS, BLK, TPS>(a, smem, slot, kb, bh);
}

// D = 256: the dV pass (PASS 1) and the dK pass (PASS 2) of every KV block in
// one launch, 2 nkb items per (b, hkv), so that the work order deals both
// passes' items longest first over the CUs together.  With one launch per
// pass each launch ends with its own tail: a windowed band puts its many
// equal-length items in the first round and the truncated ones after them
// (at config 4, 132 query tiles then 128 .. 4 per CU, against 99 on average).
// Item k of a group: KV block k / 2, the dK pass for even k (the longer of the
// two per tile: dP MFMAs and the staged dS stores) and the dV pass for odd k.
template <class T, int D, bool SOFTCAP, bool ALIBI, bool DS, bool BLK>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(KvCfg<D>::WPE, KvCfg<D>::WPE)))
void bwd_kv_passes_kernel(BwdArgs a) {
  static_assert(KvCfg<D>::PASSES, "two passes at D = 256 only");
  __shared__ __attribute__((aligned(1024))) char smem[KvCfg<D>::LDSB];
  const int nit = 2 * a.ntiles;  // items per (b, hkv)
  const int slot = queue_slot(a.queue, a.nstatic);
  if (slot >= (int)gridDim.x) return;  // (a counter that was not cleared)
  int k, bh;
  if (!xcd_lpt_item(slot, nit, a.p.B * a.p.Hkv, k, bh)) {
    const int w = xcd_remap(slot, gridDim.x);
    k = w % nit;
    bh = w / nit;
  }
  if ((k & 1) == 0) kv_tile_stream<T, D, SOFTCAP, ALIBI, DS, 2, BLK>(a, smem, slot, k >> 1, bh);
  else kv_tile_stream<T, D, SOFTCAP, ALIBI, false, 1, BLK>(a, smem, slot, k >> 1, bh);
}

#ifndef FLEXATT_KV_TPS
#define FLEXATT_KV_TPS 2  // tiles per step at D = 128 without block maps (tuning override; 1.7% faster than 1)
#endif

template <class T, int D, bool DS>
hipError_t launch_kv(const BwdArgs& a, hipStream_t st) {
  using C = KvCfg<D>;
  static_assert(C::BKV == kDsKB && C::BM == kDsQT, "staged dS units are one tile by one KV block");
  BwdArgs x = a;
  x.ntiles = (a.p.Skv + C::BKV - 1) / C::BKV;
  const dim3 grid(x.ntiles * a.p.B * a.p.Hkv), block(C::NW * 64);
  const bool sc = a.p.cap > 0.f, al = a.p.alibi != nullptr;
  auto go = [&](auto pass_c) {
    constexpr int PS = decltype(pass_c)::value;
    constexpr bool DSP = DS && PS != 1;
    x.queue = a.queue;
    // block-sparse maps: the walk list of live query tiles in dynamic LDS
    // (when it fits beside the tile stages; otherwise removed tiles are walked
    // and only their S-wave work is skipped)
    const size_t dyn = 2 * (size_t)((a.p.Sq + C::BM - 1) / C::BM + 2);
    if (a.p.blk && C::LDSB + dyn <= 160 * 1024) {
      if (sc && al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, true, DSP, PS, true>), grid, block, dyn, st, x);
      else if (sc) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, false, DSP, PS, true>), grid, block, dyn, st, x);
      else if (al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, true, DSP, PS, true>), grid, block, dyn, st, x);
      else hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, false, DSP, PS, true>), grid, block, dyn, st, x);
      return hipGetLastError();
    }
    if constexpr (D == 128 && PS == 0 && FLEXATT_KV_TPS == 2) {
      if (!a.p.blk) {
        constexpr int TP = FLEXATT_KV_TPS;
        if (sc && al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, true, DSP, PS, false, TP>), grid, block, 0, st, x);
        else if (sc) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, false, DSP, PS, false, TP>), grid, block, 0, st, x);
        else if (al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, true, DSP, PS, false, TP>), grid, block, 0, st, x);
        else hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, false, DSP, PS, false, TP>), grid, block, 0, st, x);
        return hipGetLastError();
      }
    }
    if (sc && al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, true, DSP, PS, false>), grid, block, 0, st, x);
    else if (sc) hipLaunchKernelGGL((bwd_kv_kernel<T, D, true, false, DSP, PS, false>), grid, block, 0, st, x);
    else if (al) hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, true, DSP, PS, false>), grid, block, 0, st, x);
    else hipLaunchKernelGGL((bwd_kv_kernel<T, D, false, false, DSP, PS, false>), grid, block, 0, st, x);
    return hipGetLastError();
  };
  if constexpr (C::PASSES) {
    {
      // both passes in one launch (bwd_kv_passes_kernel)
      const dim3 grid2(2 * x.ntiles * a.p.B * a.p.Hkv);
      x.queue = a.queue;
      const size_t dyn = 2 * (size_t)((a.p.Sq + C::BM - 1) / C::BM + 2);
      const bool blk = a.p.blk && C::LDSB + dyn <= 160 * 1024;
      if (blk) {
        if (sc && al) hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, true, true, DS, true>), grid2, block, dyn, st, x);
        else if (sc) hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, true, false, DS, true>), grid2, block, dyn, st, x);
        else if (al) hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, false, true, DS, true>), grid2, block, dyn, st, x);
        else hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, false, false, DS, true>), grid2, block, dyn, st, x);
      } else {
        if (sc && al) hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, true, true, DS, false>), grid2, block, 0, st, x);
        else if (sc) hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, true, false, DS, false>), grid2, block, 0, st, x);
        else if (al) hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, false, true, DS, false>), grid2, block, 0, st, x);
        else hipLaunchKernelGGL((bwd_kv_passes_kernel<T, D, false, false, DS, false>), grid2, block, 0, st, x);
      }
      return hipGetLastError();
    }
  } else {
    return go(std::integral_constant<int, 0>{});
  }
}

#define FLEXATT_KV_LAUNCHERS(D)                                                                     \
  hipError_t bwd_kv_bf16_d##D(const BwdArgs& a, hipStream_t st) { return launch_kv<__bf16, D, false>(a, st); }    \
  hipError_t bwd_kv_f16_d##D(const BwdArgs& a, hipStream_t st) { return launch_kv<_Float16, D, false>(a, st); }  \
  hipError_t bwd_kv_ds_bf16_d##D(const BwdArgs& a, hipStream_t st) { return launch_kv<__bf16, D, true>(a, st); } \
  hipError_t bwd_kv_ds_f16_d##D(const BwdArgs& a, hipStream_t st) { return launch_kv<_Float16, D, true>(a, st); }
#if FLEXATT_D == 128
FLEXATT_KV_LAUNCHERS(128)
#elif FLEXATT_D == 64
FLEXATT_KV_LAUNCHERS(64)
#else
FLEXATT_KV_LAUNCHERS(256)
#endif

#endif  // FLEXATT_D == 128 || FLEXATT_D == 64 || FLEXATT_D == 256

}  // namespace flexatt

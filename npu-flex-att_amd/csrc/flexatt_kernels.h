// Kernel argument blocks and launcher declarations (internal to libflexatt).
#pragma once
#include <hip/hip_runtime.h>

#include "flexatt_device.h"

namespace flexatt {

struct FwdArgs {
  View q, k, v;
  MutView o;
  float* lse;
  Shape p;
  int nqt;    // number of query tiles (set by the launcher)
  int gpack;  // query heads per workgroup (set by the launcher)
  int bstride;  // block-sparse maps: bytes per wave's block-map row in dynamic LDS (set by the launcher)
};

struct DeltaArgs {
  View o, dout;
  float* delta;
  int B, H, S, D;
  int* zero;  // when set: 4 queue counters the pass clears for the kernels after it
};

struct BwdArgs {
  View q, k, v, dout;
  const float* lse;
  const float* delta;
  MutView dq, dk, dv;
  Shape p;
  int ntiles;  // number of row tiles of the kernel's grid (set by the launcher)
  // dQ with Delta computed in the kernel (bwd_q only): O, and where Delta is
  // written for the dK/dV kernel; delta_out == nullptr: Delta is read from delta.
  View o;
  float* delta_out;
  // Staged dS (D = 128 fp16/bf16): the workspace the dK/dV kernel writes and
  // the dQ kernel reads, and the units stored per query head (the layout is
  // described with ds_tile_offset); ds == nullptr: not staged.
  char* ds;
  int64_t ds_head;
  // Work queue (staged path): queue == nullptr keeps the static work order;
  // otherwise workgroups from nstatic on take their slot from the counter.
  int* queue;
  int nstatic;
};

// Split-KV decode forward (fwd_decode.hip): partials in the caller's workspace.
struct DecodeArgs {
  View q, k, v;
  MutView o;
  float* lse;
  float* part_o;    // [B * Hq * Sq][nsplit][D], O of each partial / its row sums
  float* part_lse;  // [B * Hq * Sq][nsplit], LSE of each partial in log2 units
  Shape p;
  int nsplit;  // workgroups per (b, hkv)
  int chunk;   // 32-row KV tiles per workgroup
  int ntiles;  // 32-row KV tiles in the attended range
};

typedef hipError_t (*FwdLauncher)(const FwdArgs&, hipStream_t);
typedef hipError_t (*DecodeLauncher)(const DecodeArgs&, hipStream_t);
typedef hipError_t (*BwdLauncher)(const BwdArgs&, hipStream_t);

#define FLEXATT_DECL_D(D)                                                     \
  hipError_t fwd_mfma_bf16_d##D(const FwdArgs&, hipStream_t);                 \
  hipError_t fwd_mfma_f16_d##D(const FwdArgs&, hipStream_t);                  \
  hipError_t bwd_dq_mfma_bf16_d##D(const BwdArgs&, hipStream_t);              \
  hipError_t bwd_dq_mfma_f16_d##D(const BwdArgs&, hipStream_t);               \
  hipError_t bwd_dkdv_mfma_bf16_d##D(const BwdArgs&, hipStream_t);            \
  hipError_t bwd_dkdv_mfma_f16_d##D(const BwdArgs&, hipStream_t);

FLEXATT_DECL_D(32)
FLEXATT_DECL_D(64)
FLEXATT_DECL_D(128)
FLEXATT_DECL_D(256)
#undef FLEXATT_DECL_D
// D = 256 forward with wave-specialised pairs (fwd_ws.hip), called by the
// D = 256 forward launcher
hipError_t fwd_ws_bf16_d256(const FwdArgs&, hipStream_t);
hipError_t fwd_ws_f16_d256(const FwdArgs&, hipStream_t);
bool fwd_ws_fits(const Shape& p);  // its LDS (with a block map's lists) fits one CU

hipError_t bwd_delta(int dtype, const DeltaArgs&, hipStream_t);

// Split-KV decode forward (fwd_decode.hip), D <= 128.
hipError_t fwd_decode_bf16_d32(const DecodeArgs&, hipStream_t);
hipError_t fwd_decode_f16_d32(const DecodeArgs&, hipStream_t);
hipError_t fwd_decode_bf16_d64(const DecodeArgs&, hipStream_t);
hipError_t fwd_decode_f16_d64(const DecodeArgs&, hipStream_t);
hipError_t fwd_decode_bf16_d128(const DecodeArgs&, hipStream_t);
hipError_t fwd_decode_f16_d128(const DecodeArgs&, hipStream_t);

// dK/dV as a KV-stationary tile stream (bwd_kv.hip), D = 64, 128 and 256.
hipError_t bwd_kv_bf16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_f16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_bf16_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_f16_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_bf16_d256(const BwdArgs&, hipStream_t);  // dV and dK passes as items of one launch
hipError_t bwd_kv_f16_d256(const BwdArgs&, hipStream_t);

// dK/dV that also writes its dS to a.ds (bwd_kv.hip), and dQ = scale * dS K
// from it (bwd_dq_ds.hip), D = 64, 128 and 256.
hipError_t bwd_kv_ds_bf16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_f16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_bf16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_f16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_bf16_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_f16_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_bf16_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_f16_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_bf16_d256(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_f16_d256(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_bf16_d256(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_f16_d256(const BwdArgs&, hipStream_t);

// fp32 inputs on the fp32 matrix cores (f32_mfma.hip): forward, dK/dV (with
// or without writing dS), dQ from the staged dS and dQ recomputing S and dP,
// every D.
hipError_t fwd_f32_d32(const FwdArgs&, hipStream_t);
hipError_t fwd_f32_d64(const FwdArgs&, hipStream_t);
hipError_t fwd_f32_d128(const FwdArgs&, hipStream_t);
hipError_t fwd_f32_d256(const FwdArgs&, hipStream_t);
hipError_t bwd_dq_f32_d32(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_f32_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_f32_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_f32_d256(const BwdArgs&, hipStream_t);
hipError_t bwd_dkdv_f32_d32(const BwdArgs&, hipStream_t);
hipError_t bwd_dkdv_f32_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_dkdv_f32_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_dkdv_f32_d256(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_f32_d32(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_f32_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_f32_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_kv_ds_f32_d256(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_f32_d32(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_f32_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_f32_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_dq_ds_f32_d256(const BwdArgs&, hipStream_t);

// dQ as a query-stationary tile stream (bwd_q.hip), D = 64 and 128; with
// a.delta_out set it also computes Delta (written there) from O and dO.
hipError_t bwd_q_bf16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_q_f16_d128(const BwdArgs&, hipStream_t);
hipError_t bwd_q_bf16_d64(const BwdArgs&, hipStream_t);
hipError_t bwd_q_f16_d64(const BwdArgs&, hipStream_t);

}  // namespace flexatt

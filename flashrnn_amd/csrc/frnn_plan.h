// The launch plan shared by the host launcher and the kernels.
//
// A plan fixes, for one (cell, B, T, N, D, dtype, mma) problem:
//  * the batch slab of a group (16*NB rows) and the number of slabs;
//  * KS, the waves per workgroup that split the contraction dimension;
//  * the workgroup -> (group, hidden tile) map that keeps a group on one XCD;
//  * the sizes and offsets of every caller-owned area.
// Forward and backward of one problem use the same plan, so the
// saved-for-backward area can be laid out exactly as the lanes own it.
#pragma once

#include <stdint.h>

namespace frnn {

constexpr int kXcds = 8;      // MI355X: 8 XCDs, workgroup w is dispatched to XCD w % 8
constexpr int kMaxKT = 8;     // max 32-wide k-tiles per gate and wave (forward)
constexpr int kMaxNFB = 32;   // max 32-wide k-tiles per wave (backward)
// Plan flags (the C ABI's frnn_flags)
constexpr int kFlagTraining = 1, kFlagShared = 2, kFlagCut = 4, kFlagClip = 8, kFlagUnready = 16;
constexpr int kFlagOutHidden = 32, kFlagOutLast = 64, kFlagSnapF32 = 128, kFlagV1Grad = 256;
// Launch-internal flag (never set by a caller): one more workgroup per group
// (XCD-local mode, backward), the group's scout, that touches the inputs of
// later steps so they wait in the XCD's L2.
constexpr int kFlagScout = 1 << 20;

struct Plan {
  int cell, B, T, N, D;
  int GR, GW, GT, S;
  int mma, dt_io, dt_state, flags;
  float clip;      // kFlagClip: clamp bound of h and of its recurrent cotangent
  int Ttot, t0;    // forward step window: Wx and the outputs hold Ttot steps, this call runs
                   // steps [t0, t0 + T) of them (Ttot == T, t0 == 0 for a whole sequence)
  int dt_out;      // dtype of the state output (dt_io, or FP32 with kFlagSnapF32)
  int dt_save;     // dtype of the saved-for-backward values: FP16 with 16-bit MMA operands
                   // (LSTM, GRU, Elman), FP32 otherwise
  int NB;          // 16-row batch tiles per group
  int BS;          // slab rows = 16 * NB
  int nslab;       // ceil(B / BS)
  int ngroups;     // N * nslab
  int wpg;         // workgroups per group = D / (16 * NDT)
  int KS;          // forward: compute waves per hidden tile (contraction split)
  int KSB;         // backward: compute waves per hidden tile
  int NDT;         // hidden tiles per workgroup (workgroup = NDT * KS waves)
  int grid;        // launched workgroups of one launch (idle ones exit at once)
  int g0, gcount;  // groups [g0, g0 + gcount) run in this launch (launches run in turn when
                   // all groups cannot be resident at once; groups never wait on each other)
  int nwg;         // active workgroups = ngroups * wpg
  int kt_fwd;      // D / 32
  int kt_bwd;      // GR * D / 32
  int epl;         // owned elements per lane = ceil(4 * NB / KS)
  int nsave;       // saved floats per owned element and step
  // byte sizes / offsets
  long long xwords_fwd, xwords_bwd;   // exchange words per parity
  long long save_floats;              // lane-native saved values
  int splitk;                         // dR GEMM split over K
  long long ws_fwd, ws_bwd, save_bytes;
  long long off_dcand;                // backward workspace: GRU candidate-gate cotangents
  long long off_x, off_flag;          // workspace offsets (status word at 0)
  long long off_claim_f, off_claim_b; // workgroup slot counters: 8 per launch (one per XCD), by first group
  long long off_part, off_dbpart;     // backward: dR split-K partials, db partials
  int dma_gemm;                       // backward: the dR GEMM runs on the LDS-DMA kernel
};

// Group / tile of a workgroup; returns false for an idle workgroup.
//  * placement-free exchange: workgroup index wg in a compact grid;
//  * XCD-local exchange: wg is the workgroup's claim on its XCD (the
//    workgroups that run on XCD x number themselves 0, 1, ... in arrival
//    order), and groups x, x + 8, x + 16, ... of the launch live on XCD x.
#if defined(__HIPCC__)
__host__ __device__
#endif
inline bool wg_decode(const Plan& p, int wg, int xcd, int* group, int* member) {
  int local;
  if (p.flags & 2) {
    local = wg / p.wpg;
    *member = wg % p.wpg;
  } else {
    const int slot = wg / p.wpg;
    *member = wg % p.wpg;
    local = slot * kXcds + xcd;
  }
  *group = p.g0 + local;
  return local < p.gcount;
}

// Scouts (kFlagScout, XCD-local exchange only) are the last 8 * ceil(gcount / 8)
// workgroups of a launch's grid, after the members' slots; each claims, on its
// own counters, the next group of the XCD it runs on.
#if defined(__HIPCC__)
__host__ __device__
#endif
inline int scout_blocks(const Plan& p) {
  return (p.flags & kFlagScout) ? kXcds * ((p.gcount + kXcds - 1) / kXcds) : 0;
}

}  // namespace frnn

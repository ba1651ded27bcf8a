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

#include <stddef.h>
#include <stdint.h>

struct frnn_desc;

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
  int rs;                             // backward: reduce-scatter exchange (bwd_rs_kernel)
  int ptm;                            // reduce-scatter: output tiles per compute wave (class)
  int nscout;                         // scouts per group in a launch with kFlagScout (>= 1)
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

// Scouts (kFlagScout, XCD-local exchange only) are the last
// 8 * ceil(gcount / 8) * nscout workgroups of a launch's grid, after the
// members' slots; each claims, on its own counters, the next slot of the XCD
// it runs on: slot / nscout is the group (of that XCD), slot % nscout the
// scout's share of the group's touches.
#if defined(__HIPCC__)
__host__ __device__
#endif
inline int scout_blocks(const Plan& p) {
  return (p.flags & kFlagScout) ? kXcds * ((p.gcount + kXcds - 1) / kXcds) * (p.nscout > 1 ? p.nscout : 1) : 0;
}

// ---------------------------------------------------------------- addressing
// Index arithmetic of the kernels' global and exchange accesses, shared with
// the host bounds check (tests/bounds): every element or word a kernel touches
// is computed by one of these functions.
#if defined(__HIPCC__)
#define FRNN_HD __host__ __device__
#else
#define FRNN_HD
#endif

// I/O lane `lane`, its i-th element: e = 256*(i/4) + 4*lane + i%4 (four
// consecutive hidden units of one batch row per lane and batch tile).
FRNN_HD inline int io_elem(int lane, int i) { return 256 * (i >> 2) + 4 * lane + (i & 3); }

// Element e of hidden tile dt of slab `slab` -> hidden unit d, slab row bl, batch row b.
struct ElemPos {
  int d, bl, b;
  bool real;
};
FRNN_HD inline ElemPos elem_pos(const Plan& p, int slab, int dt, int e) {
  ElemPos x;
  const int bt = e >> 8, r = e & 255;
  x.d = dt * 16 + (r & 15);
  x.bl = bt * 16 + (r >> 4);
  x.b = slab * p.BS + x.bl;
  x.real = x.b < p.B;
  return x;
}

// Forward I/O lane's Wx DMA of window step u, gate g: element index of the
// first of the 16 bytes it reads (4 FP32 or 8 16-bit units of one row), and
// whether the lane reads at all (real row; 16-bit rows use the even quads).
FRNN_HD inline long wx_dma_index(const Plan& p, int slab, int n, int dt, int lane, int u, int g, int esz, bool* valid) {
  const int lrow = lane >> 2, lquad = lane & 3;
  const int lb = slab * p.BS + lrow;
  *valid = lb < p.B && (esz == 4 || (lquad & 1) == 0);
  const long wx_t = (long)p.GW * p.N * p.D;
  return ((long)lb * p.Ttot + p.t0 + u) * wx_t + ((long)g * p.N + n) * p.D + dt * 16 + 4 * lquad;
}

// State k of batch row b at window step t, head n, unit d: index into the
// state output [nst][B][Ttot][N][D].
FRNN_HD inline long state_index(const Plan& p, int k, int b, int t, int n, int d) {
  return ((((long)k * p.B + b) * p.Ttot + p.t0 + t) * p.N + n) * p.D + d;
}
// The FRNN_OUT_LAST output [B][1][N][D].
FRNN_HD inline long last_index(const Plan& p, int b, int n, int d) { return ((long)b * p.N + n) * p.D + d; }
// Initial state / carry / their cotangents [S][B][N][D].
FRNN_HD inline long carry_index(const Plan& p, int k, int b, int n, int d) {
  return (((long)k * p.B + b) * p.N + n) * p.D + d;
}

// Lane-native saved values: [t][workgroup][value][team*NE + e].
FRNN_HD inline long save_index(const Plan& p, int ne, int t, int wgi, int v, int team, int e) {
  const long per = (long)p.NDT * ne;
  return (((long)t * p.nwg + wgi) * p.nsave + v) * per + (long)team * ne + e;
}

// Backward scout: touch slots of one step for a group (state-cotangent lines,
// nst values of nreal rows at esz bytes; then every 128-byte line of the
// group's saved values at ssz bytes), shared out among the group's scouts.
FRNN_HD inline int bwd_scout_lines(const Plan& p, int nst, int nreal, int esz, int ssz) {
  const int lpr = (p.D * esz + 127) / 128 + 1;  // lines of one row (+1: unaligned rows)
  return nst * nreal * lpr + p.wpg * p.nsave * p.NDT * p.NB * 2 * ssz;
}

// Exchange word of (row r, contraction index k) in one group's table, chunk-major
// with wp words per 16-byte chunk (see XLayout in frnn_device.h).
FRNN_HD inline int xword_rt(int wp, int BS, int r, int k) {
  const int nc = 8 / wp;
  const int kt = k >> 5, kq = (k >> 3) & 3, c = (k & 7) / wp, e = k % wp;
  return (((kt * 4 + kq) * nc + c) * BS + r) * wp + e;
}

// Forward scout touch: byte offset into Wx of line l of (slab row r, window
// step u, gate g); a row's lines are clamped to its last 4 bytes.
FRNN_HD inline long scout_wx_byte(const Plan& p, int slab, int n, int r, int u, int g, int l, int esz) {
  const long e0 = ((((long)(slab * p.BS + r) * p.Ttot + p.t0 + u) * p.GW + g) * p.N + n) * p.D;
  const int row_bytes = p.D * esz;
  return e0 * esz + (128 * l < row_bytes - 4 ? 128 * l : row_bytes - 4);
}

}  // namespace frnn

// Test hook of libfrnn.so (not part of the public ABI in include/frnn.h): copies
// the launch plan of *d (a frnn_desc) into plan_out (bytes == sizeof(frnn::Plan)),
// for the host bounds check; returns make_plan's code.
extern "C" int frnn_test_plan(const struct frnn_desc* d, void* plan_out, size_t bytes);

// Kernel argument blocks and kernel lookup, shared by the kernels and the launcher.
#pragma once

#include <stdint.h>

#include "frnn_plan.h"

namespace frnn {

// Input projection workers (frnn_proj.h): Wx[B][T][ncols] = x[B][T][I] W[ncols][I]^T
// in 128 x 128 tiles of output rows m = t*B + b and columns.
constexpr int kProjRows = 128, kProjCols = 128;

struct ProjArgs {
  const void* x;     // [B][T][I]
  const void* w;     // [ncols][I]
  void* wx;          // [B][T][ncols]
  uint32_t* ready;   // [nrt]: column tiles done per row tile (zeroed before the launch)
  uint32_t* next;    // tile counter (zeroed before the launch)
  int I, ncols;      // inner size (multiple of 8), G_W*N*D (multiple of 32)
  int B, T;
  int nrt, nct;      // row tiles ceil(B*T/128), column tiles ceil(ncols/128)
  uint32_t skip_xcds;  // beside the recurrence: XCDs whose workers leave at once (bit per XCD)
  int plain;           // beside the recurrence: the recurrence reads Wx with plain (L2-cached) loads
};

// Last row tile that step t of the sequence reads: rows t*B .. t*B+B-1.
#ifdef __HIPCC__
__host__ __device__
#endif
inline int proj_last_row_tile(int t, int B) { return (int)(((long)(t + 1) * B - 1) / kProjRows); }

// Element indices the projection workers address (frnn_proj.h), shared with
// the host bounds check (tests/bounds/proj_bounds.cpp). Rows past B*T read x
// row 0 and columns past ncols read W row 0 (their products are never
// stored); an 8-run whose k lies past I reads k 0 of its row instead (masked
// out of the products), so every address stays inside its operand.
FRNN_HD inline long proj_x_row(const ProjArgs& pa, long m) {
  const long rows = (long)pa.B * pa.T, mm = m < rows ? m : 0;
  return ((mm % pa.B) * pa.T + mm / pa.B) * pa.I;
}
FRNN_HD inline long proj_w_row(const ProjArgs& pa, int c) { return (long)(c < pa.ncols ? c : 0) * pa.I; }
FRNN_HD inline int proj_k8(const ProjArgs& pa, int k8) { return k8 < pa.I ? k8 : 0; }
FRNN_HD inline long proj_wx_elem(const ProjArgs& pa, long m, int c) {
  return ((m % pa.B) * pa.T + m / pa.B) * pa.ncols + c;
}

struct FwdArgs {
  Plan p;
  const void* wx;
  const void* R;
  const void* bias;
  const void* s0;
  void* states;
  void* carry;
  void* save;               // lane-native saved values (training, dtype p.dt_save) or null
  char* xbuf;               // exchange, both parities
  long long xbytes;
  uint32_t* claim;          // zeroed slot counters (XCD-local exchange)
  uint32_t* status;
  uint32_t spin_limit;
  unsigned long long* prof;  // phase profile (8 words) or null
  ProjArgs proj;             // projection-gated launches only: the producers' arguments
};

struct BwdArgs {
  Plan p;
  const void* R;
  const void* save;         // lane-native saved values (dtype p.dt_save)
  const void* s0;           // initial states [S][B][N][D] (dtype p.dt_state): the sLSTM's c_{-1}, n_{-1}
  const void* d_states;     // may be null
  const void* d_carry;      // may be null
  void* dwx;
  void* ds0;
  float* dcand;             // GRU: cotangent of the R-only candidate gate [B,T,N,D] (dR GEMM operand)
  float* dbpart;
  char* xbuf;
  long long xbytes;
  uint32_t* claim;          // zeroed slot counters (XCD-local exchange)
  uint32_t* status;
  uint32_t spin_limit;
  unsigned long long* prof;  // phase profile (8 words, after the forward's 8) or null
};

// dR[g,n,o,p] = sum over (b,t) of dG[b,t,g,n,o] h_{t-1}[b,n,p], read from the
// public dWx (GRU: gate 0 from dcand) and the forward's state output (h_{-1} = s0).
struct GemmArgs {
  Plan p;
  const void* dwx;
  const float* dcand;
  const void* states;
  const void* s0;
  float* part;
  const float* dbpart;
  void* dR;
  void* db;
  const void* zero;     // 256 zero bytes (the DMA path's source for k beyond B*T)
  const void* dcand16;  // GRU, DMA path: dcand in the MMA type
};

// dR GEMM whose operand tiles are loaded by LDS-DMA several stages ahead: 16-bit
// operands in the MMA's type (dWx, states and s0 alike; the GRU's candidate gate
// from its 16-bit copy dcand16), D % 64 == 0; null otherwise.
const void* gemm_dma_kernel(int mma);
// FP32 -> 16-bit copy (the DMA GEMM's h_{-1} rows when s0 is FP32).
const void* to16_kernel();

// Persistent recurrence kernel for (mma, k-tiles per wave) of one cell; null if not built.
// proj: the forward that also runs the input-projection workers (frnn_proj.h).
const void* lstm_kernel(int mma, int ks, int ktw, int ndt, bool forward, bool proj = false);
const void* gru_kernel(int mma, int ks, int ktw, int ndt, bool forward, bool proj = false);
const void* elman_kernel(int mma, int ks, int ktw, int ndt, bool forward, bool proj = false);
const void* slstm_kernel(int mma, int ks, int ktw, int ndt, bool forward, bool proj = false);
// LDS floats per hidden-tile team of the persistent kernels (KS compute waves).
long lstm_lds_floats(bool forward, int ks);
long gru_lds_floats(bool forward, int ks);
long elman_lds_floats(bool forward, int ks);
long slstm_lds_floats(bool forward, int ks);

inline long recurrence_lds_floats(int cell, bool forward, int ks) {
  switch (cell) {
    case 0: return lstm_lds_floats(forward, ks);
    case 1: return gru_lds_floats(forward, ks);
    case 2: return elman_lds_floats(forward, ks);
    case 3: return slstm_lds_floats(forward, ks);
  }
  return 0;
}

inline const void* recurrence_kernel(int cell, int mma, int ks, int ktw, int ndt, bool forward, bool proj = false) {
  switch (cell) {
    case 0: return lstm_kernel(mma, ks, ktw, ndt, forward, proj);
    case 1: return gru_kernel(mma, ks, ktw, ndt, forward, proj);
    case 2: return elman_kernel(mma, ks, ktw, ndt, forward, proj);
    case 3: return slstm_kernel(mma, ks, ktw, ndt, forward, proj);
  }
  return nullptr;
}
// Reduce-scatter backward kernels (frnn_bwd_rs.h) for (mma, hidden tiles per
// workgroup, compute waves per tile, output-tile class); null if not built.
const void* lstm_rs_kernel(int mma, int ndt, int ks, int ptm);
const void* gru_rs_kernel(int mma, int ndt, int ks, int ptm);
const void* elman_rs_kernel(int mma, int ndt, int ks, int ptm);
const void* slstm_rs_kernel(int mma, int ndt, int ks, int ptm);
long lstm_rs_lds_floats(int ndt);
long gru_rs_lds_floats(int ndt);
long elman_rs_lds_floats(int ndt);
long slstm_rs_lds_floats(int ndt);
inline const void* rs_kernel(int cell, int mma, int ndt, int ks, int ptm) {
  switch (cell) {
    case 0: return lstm_rs_kernel(mma, ndt, ks, ptm);
    case 1: return gru_rs_kernel(mma, ndt, ks, ptm);
    case 2: return elman_rs_kernel(mma, ndt, ks, ptm);
    case 3: return slstm_rs_kernel(mma, ndt, ks, ptm);
  }
  return nullptr;
}
inline long rs_lds_floats(int cell, int ndt) {
  switch (cell) {
    case 0: return lstm_rs_lds_floats(ndt);
    case 1: return gru_rs_lds_floats(ndt);
    case 2: return elman_rs_lds_floats(ndt);
    case 3: return slstm_rs_lds_floats(ndt);
  }
  return 0;
}

// dR GEMM: wide = 64x64 workgroup tiles (4 waves, D % 64 == 0), else 32x32 (1 wave).
const void* gemm_kernel(int mma, bool wide);
// Input-projection workers alone (frnn_proj.h), 256 threads and proj_lds_bytes() of
// dynamic LDS: 16-bit MMA types; null otherwise.
const void* proj_kernel(int mma);
int proj_lds_bytes();
const void* reduce_kernel();
const void* zero_kernel();

}  // namespace frnn

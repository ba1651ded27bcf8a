// C ABI of libfrnn.so: validation, launch plan, workspace layout, launches.
// Replaces FlashRNNFuncFused (flashrnn/flashrnn/fused/flashrnn.cc:244-535)
// and ForwardPass/BackwardPass::Run (fused/flashrnn_fused_forward.cu:773-976,
// fused/flashrnn_fused_backward.cu:769-1087). See include/frnn.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/frnn.h"
#include "frnn_kernels.h"
#include "frnn_plan.h"

namespace {

using frnn::Plan;

constexpr uint32_t kDefaultSpinLimit = 1u << 22;
std::atomic<uint32_t> g_spin_limit{kDefaultSpinLimit};
// FRNN_NO_GEMM_DMA=1 (environment, read once): the dR GEMM's register-staged kernel only.
std::atomic<bool> g_no_gemm_dma{[] {
  const char* e = std::getenv("FRNN_NO_GEMM_DMA");
  return e && *e && *e != '0';
}()};
// FRNN_NO_SCOUT=1 (environment, read once): no L2-prefetch workgroups in the backward.
std::atomic<bool> g_no_scout{[] {
  const char* e = std::getenv("FRNN_NO_SCOUT");
  return e && *e && *e != '0';
}()};
std::atomic<unsigned long long*> g_phase_prof{nullptr};

// ---- optional kernel timing (frnn_timing_enable / frnn_timing_read)
struct Timing {
  std::mutex mu;
  bool on = false;
  std::vector<hipEvent_t> free_events;
  struct Rec { int kind; hipEvent_t a, b; };
  std::vector<Rec> pending;
  hipEvent_t get() {
    if (!free_events.empty()) {
      hipEvent_t e = free_events.back();
      free_events.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
Timing g_timing;

// Record the start event of a timed region; returns false when timing is off.
bool timing_begin(hipStream_t st, hipEvent_t* a) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  if (!g_timing.on) return false;
  *a = g_timing.get();
  return *a && hipEventRecord(*a, st) == hipSuccess;
}
void timing_end(int kind, hipEvent_t a, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  hipEvent_t b = g_timing.get();
  if (!b || hipEventRecord(b, st) != hipSuccess) return;
  g_timing.pending.push_back({kind, a, b});
}

constexpr long long kAlign = 256;
long long align_up(long long x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool cell_sizes(int cell, int* gr, int* gw, int* gt, int* s) {
  switch (cell) {
    case FRNN_LSTM: *gr = 4; *gw = 4; *gt = 4; *s = 2; return true;
    case FRNN_GRU: *gr = 3; *gw = 3; *gt = 4; *s = 1; return true;
    case FRNN_ELMAN: *gr = 1; *gw = 1; *gt = 1; *s = 1; return true;
    case FRNN_SLSTM: *gr = 4; *gw = 4; *gt = 4; *s = 4; return true;
  }
  return false;
}

int nsave_of(int cell) {
  switch (cell) {
    case FRNN_LSTM: return 6;
    case FRNN_GRU: return 5;
    case FRNN_ELMAN: return 1;
    case FRNN_SLSTM: return 8;
  }
  return 0;
}

// Smallest built k-tiles-per-wave class that holds `need` for a workgroup of
// `ndt` hidden tiles (one-tile workgroups: 1, 2, 4; two-tile: 6, 8).
int ktw_class(int need, int ndt) {
  if (ndt == 1) {
    for (int c : {1, 2, 4})
      if (need <= c) return c;
  } else {
    for (int c : {6, 8})
      if (need <= c) return c;
  }
  return 0;
}

// Whether a wave of a workgroup with `ks` compute waves per hidden tile holds
// its resident R (forward) or R^T (backward) slice plus the exchange runs it
// keeps in flight (at most 8 BF16 runs in one-tile workgroups, else 4) in its
// share of the register file: the 512 registers of a SIMD lane divided among
// the waves per SIMD, less 56 for the rest of the loop. The variant must also
// be built.
bool fits(const Plan& p, int ks, bool forward) {
  const int need = (p.kt_fwd + ks - 1) / ks;
  const int ktw = ktw_class(need, p.NDT);
  if (!ktw || !frnn::recurrence_kernel(p.cell, p.mma, ks, ktw, p.NDT, forward)) return false;
  if (p.NDT == 2 && ks != 3 && ks != 4) return false;
  const int waves = p.NDT * (ks + 1);
  const int per_simd = (waves + 3) / 4;
  const int budget = (512 / per_simd) / 8 * 8 - 56;
  const int frag = p.mma == FRNN_MMA_F32 ? 8 : 4;  // registers of one resident fragment
  const int run = 2 * frag;                         // registers of one in-flight exchange run
  const int frags = p.GR * ktw;
  const int runs = std::min(forward ? ktw : frags, (p.mma != FRNN_MMA_F32 && p.NDT == 1) ? 8 : 4);
  return frags * frag + runs * run <= budget;
}

// Groups [g0, g0 + n) form one launch; its grid in either placement mode.
void set_groups(Plan* p, int g0, int n) {
  p->g0 = g0;
  p->gcount = n;
  p->grid = (p->flags & FRNN_XCD_SHARED) ? n * p->wpg
                                          : frnn::kXcds * p->wpg * ((n + frnn::kXcds - 1) / frnn::kXcds) +
                                                frnn::scout_blocks(*p);
}

// MMA-type dtype of a 16-bit policy, or -1 (FP32 operands).
int mma_h16(int mma) { return mma == FRNN_MMA_BF16 ? FRNN_BF16 : (mma == FRNN_MMA_F16 ? FRNN_F16 : -1); }

// Whether the backward's dR GEMM runs on the LDS-DMA kernel: 16-bit operands
// already in the MMA's type (dWx and the state history; s0 in that type or FP32),
// 64-wide tiles, and the kernel not switched off.
bool gemm_uses_dma(const Plan& p) {
  const int h16 = mma_h16(p.mma);
  return p.D % 64 == 0 && h16 >= 0 && p.dt_io == h16 && p.dt_out == h16 &&
         (p.dt_state == h16 || p.dt_state == FRNN_F32) && !g_no_gemm_dma.load();
}

// Bytes at the end of the backward workspace, for the LDS-DMA dR GEMM only: a
// 16-bit copy of an FP32 s0[0] ([B][N][D]) and, for the GRU, of the FP32
// candidate-gate cotangents ([B][T][N][D]).
long long s0_copy_bytes(const Plan& p) {
  return p.dma_gemm && p.dt_state == FRNN_F32 ? align_up((long long)p.B * p.N * p.D * 2) : 0;
}
long long cand_copy_bytes(const Plan& p) {
  return p.dma_gemm && p.cell == FRNN_GRU ? align_up((long long)p.B * p.T * p.N * p.D * 2) : 0;
}

int make_plan(const frnn_desc* d, Plan* p) {
  if (!d) return FRNN_E_INVALID;
  std::memset(p, 0, sizeof(*p));
  if (!cell_sizes(d->cell, &p->GR, &p->GW, &p->GT, &p->S)) return FRNN_E_INVALID;
  if (d->batch < 1 || d->steps < 1 || d->heads < 1 || d->width < 1) return FRNN_E_INVALID;
  if (d->dtype_io != FRNN_F32 && d->dtype_io != FRNN_BF16 && d->dtype_io != FRNN_F16) return FRNN_E_INVALID;
  if (d->dtype_state != FRNN_F32 && d->dtype_state != FRNN_BF16 && d->dtype_state != FRNN_F16)
    return FRNN_E_INVALID;
  if (d->mma != FRNN_MMA_BF16 && d->mma != FRNN_MMA_F32 && d->mma != FRNN_MMA_F16) return FRNN_E_INVALID;
  if (d->width % 32 != 0 || d->width > 1024) return FRNN_E_UNSUPPORTED;
  p->cell = d->cell;
  p->B = d->batch;
  p->T = d->steps;
  p->N = d->heads;
  p->D = d->width;
  p->mma = d->mma;
  p->dt_io = d->dtype_io;
  p->dt_state = d->dtype_state;
  p->flags = d->flags;
  if (d->flags & ~(FRNN_TRAINING | FRNN_XCD_SHARED | FRNN_GRAD_CUT | FRNN_GRAD_CLIP | FRNN_TEST_UNREADY |
                   FRNN_OUT_HIDDEN | FRNN_OUT_LAST | FRNN_SNAPSHOT_F32 | FRNN_SLSTM_V1GRAD))
    return FRNN_E_INVALID;
  if ((d->flags & FRNN_OUT_HIDDEN) && (d->flags & FRNN_OUT_LAST)) return FRNN_E_INVALID;
  p->Ttot = d->total_steps == 0 ? d->steps : d->total_steps;
  p->t0 = d->step_base;
  if (p->t0 < 0 || p->Ttot < 1 || (long long)p->t0 + d->steps > p->Ttot) return FRNN_E_INVALID;
  p->dt_out = (d->flags & FRNN_SNAPSHOT_F32) ? FRNN_F32 : d->dtype_io;
  // saved-for-backward values: FP16 under the 16-bit operand policies (every value
  // the LSTM, GRU and Elman save is an activation in [-1, 1], a state or a gate
  // pre-activation, |x| < 65504; FP16 keeps 11 significant bits), FP32 with FP32
  // operands (1e-4 parity) and for the sLSTM (its gradient is ill-conditioned at a
  // zero start, and its normalizer state grows with the sequence)
  p->dt_save = (d->mma != FRNN_MMA_F32 && d->cell != FRNN_SLSTM) ? FRNN_F16 : FRNN_F32;
  // the backward needs the hidden-state history of the whole sequence (its dR GEMM operand)
  if ((d->flags & FRNN_TRAINING) && ((d->flags & FRNN_OUT_LAST) || p->Ttot != d->steps)) return FRNN_E_UNSUPPORTED;
  if (d->flags & FRNN_GRAD_CLIP) {
    if (!(d->clipval >= 0.f) || d->clipval > 3.4e38f) return FRNN_E_INVALID;  // NaN, negative or infinite
    p->clip = d->clipval;
  }
  p->NB = 1;
  p->BS = 16 * p->NB;
  p->nslab = (p->B + p->BS - 1) / p->BS;
  p->ngroups = p->N * p->nslab;
    p->kt_fwd = p->D / 32;
  p->kt_bwd = p->GR * p->D / 32;
  const int KT = p->kt_fwd;
  // hidden tiles per workgroup: a group must fit the 32 CUs of one XCD
  p->NDT = (p->D / 16 <= 32) ? 1 : 2;
  // FRNN_NDT=2 (environment, read per plan): two hidden tiles per workgroup at any
  // width with an even tile count (half the workgroups per group)
  if (const char* e = std::getenv("FRNN_NDT"))
    if (std::atoi(e) == 2 && (p->D / 16) % 2 == 0) p->NDT = 2;
  // contraction split (compute waves per hidden tile, plus one I/O wave):
  // forward 4 (two-tile workgroups: up to 4); backward up to 8 where D/32 >= 8
  // (its exchange operand is GR times wider, so splitting it further shortens
  // each wave's poll). Two-tile
  // workgroups whose resident R slice does not fit beside 4 waves per tile use 3
  // (8 waves: two per SIMD, 256 registers each). FRNN_KS / FRNN_KS_BWD
  // (environment, read per plan) override within the built set.
  // One-tile workgroups take four compute waves also where D/32 < 4: the
  // waves without k-tiles poll nothing and add a zero partial, and the 256
  // elements of the tile are spread one per lane instead of 2-4 (measured at
  // B16 T1024: D32 forward 1.43 -> 1.17 ms, D64 1.23 -> 1.19 ms).
  p->KS = (KT >= 4 || p->NDT == 1) ? 4 : (KT >= 2 ? 2 : 1);
  // eight from D384 (each wave would otherwise poll three or more k-tiles), and
  // at D256 with more than 8 batch rows (measured, forward: LSTM B16 T1024
  // D512 2.31 -> 1.86 ms, D384 1.83 -> 1.47 ms, B8 D384 1.64 -> 1.32 ms;
  // B16 D256 GRU 0.66 -> 0.58, Elman 0.64 -> 0.53, LSTM 1.39 -> 1.37 ms;
  // but at B <= 8 and D256 every cell was 2-10% slower)
  if (p->NDT == 1 && (KT >= 12 || (KT >= 8 && p->B > 8)) && fits(*p, 8, true)) p->KS = 8;
  if (p->NDT == 1 && KT < 4 && !fits(*p, 4, true)) p->KS = KT >= 2 ? 2 : 1;
  if (p->NDT == 2 && !fits(*p, 4, true)) p->KS = 3;
  // (also where the backward's operand alone is wide: G_R*D/32 >= 16, LSTM
  // B16 T1024 D128 backward 1.86 -> 1.54 ms; at D64, 8 k-tiles, it was slower)
  p->KSB = ((KT >= 8 || p->kt_bwd >= 16) && p->NDT == 1) ? 8 : p->KS;
  if (p->NDT == 1 && p->KSB == 8 && !fits(*p, 8, false)) p->KSB = 4;
  if (p->NDT == 2 && !fits(*p, p->KSB, false)) p->KSB = 3;
  // two-tile workgroups whose reduce-scatter backward is built with four compute
  // waves per tile (the GRU; up to 48 tiles: six output tiles a wave) take it:
  // every SIMD then runs two of the eight compute waves' MFMAs (GRU B16 T512
  // D768 backward 3.10 -> 2.48 ms, D640 3.00 -> 2.33 ms; the LSTM's spilled)
  {
    const char* e = std::getenv("FRNN_BWD_RS");
    if (p->NDT == 2 && p->D / 16 <= 48 && !(e && *e == '0') && frnn::rs_kernel(p->cell, p->mma, 2, 4, 6))
      p->KSB = 4;
  }
  auto ks_env = [&](const char* name, int* ks) {
    if (const char* e = std::getenv(name)) {
      const int v = std::atoi(e);
      if ((v == 1 || v == 2 || v == 4 || (v == 8 && p->NDT == 1) || (v == 3 && p->NDT == 2)) && (v <= KT || v <= 4 || (v == 8 && KT >= 4)))
        *ks = v;
    }
  };
  ks_env("FRNN_KS", &p->KS);
  ks_env("FRNN_KS_BWD", &p->KSB);
  if (!fits(*p, p->KS, true)) return FRNN_E_UNSUPPORTED;
  p->epl = (4 * p->NB + p->KS - 1) / p->KS;
  p->nsave = nsave_of(p->cell);
  p->wpg = p->D / (16 * p->NDT);
  set_groups(p, 0, p->ngroups);
  p->nwg = p->ngroups * p->wpg;
  const long long wsz = p->mma == FRNN_MMA_F32 ? 8 : 4;
  p->xwords_fwd = (long long)p->ngroups * p->BS * p->D;
  p->xwords_bwd = (long long)p->ngroups * p->BS * p->GR * p->D;
  // Reduce-scatter backward (frnn_bwd_rs.h) for two-tile workgroups, where it is
  // built: measured at B16 T1024 D768 it takes the LSTM backward from 16.2 to
  // 8.6 ms and the GRU's (T512) from 5.0 to 4.4 ms, while at one-tile widths it
  // is 2-3x slower than the all-gather (B8 T1024 N3 D256: 4.1 against 1.6 ms).
  // FRNN_BWD_RS=0 (environment, read per plan) keeps the all-gather. Its table
  // holds D * 16 * wpg 32-bit words per group and parity.
  {
    const int ntile = p->D / 16, ncw = p->NDT * p->KSB;
    const int need = (ntile + ncw - 1) / ncw;
    p->ptm = 0;  // the smallest built class that covers the need
    for (int c : {2, 4, 6, 8, 16})
      if (!p->ptm && need <= c && frnn::rs_kernel(p->cell, p->mma, p->NDT, p->KSB, c)) p->ptm = c;
    const char* e = std::getenv("FRNN_BWD_RS");
    const bool off = e && *e == '0';
    p->rs = (!off && p->NDT == 2 && p->ptm && p->wpg <= p->ptm * p->KSB &&
             frnn::rs_kernel(p->cell, p->mma, p->NDT, p->KSB, p->ptm) != nullptr) ? 1 : 0;
    if (p->rs) p->xwords_bwd = (long long)p->ngroups * p->D * 16 * p->wpg;
  }
  if (!p->rs && !fits(*p, p->KSB, false)) return FRNN_E_UNSUPPORTED;
  p->save_floats = (long long)p->T * p->nwg * p->nsave * p->NDT * 256 * p->NB;
  // dR GEMM: 64x64 workgroup tiles where D % 64 == 0 (else 32x32), split over
  // K = B*T to fill the GPU (~2048 workgroups, >= 8 k-steps of 32 each): the
  // GEMM is bound by its operand-load latency, so more workgroups in flight
  // pay for the larger split-K reduction (measured at B8 T1024 N3 D256 and at
  // B256 T1024 N8 D128 with the LDS-DMA GEMM: 1024, 2048 and 4096 workgroups)
  const int tile = p->D % 64 == 0 ? 64 : 32;
  const long long tiles = (long long)p->N * (p->GR * p->D / tile) * (p->D / tile);
  const long long ktt = ((long long)p->B * p->T + 31) / 32;
  long long split = std::max<long long>(1, 2048 / std::max<long long>(1, tiles));
  split = std::min<long long>(split, std::max<long long>(1, ktt / 8));
  p->splitk = (int)std::min<long long>(split, 64);
  // saved-for-backward area: the lane-native values only
  p->save_bytes = align_up(p->save_floats * (p->dt_save == FRNN_F32 ? 4 : 2));
  // workspaces: status word at 0, exchange at 256
  p->off_x = kAlign;
  // by a launch's first group: the members' counters, then the scouts'
  const long long nclaim = 2LL * p->ngroups * frnn::kXcds * 4;
  p->off_claim_f = align_up(p->off_x + 2 * p->xwords_fwd * wsz);
  p->ws_fwd = align_up(p->off_claim_f + nclaim);
  p->off_claim_b = align_up(p->off_x + 2 * p->xwords_bwd * (p->rs ? 4 : wsz));
  p->off_dcand = align_up(p->off_claim_b + nclaim + 256);  // + 256 zero bytes (dR GEMM's DMA tail source)
  const long long ndcand = p->cell == FRNN_GRU ? (long long)p->B * p->T * p->N * p->D : 0;
  p->off_part = align_up(p->off_dcand + ndcand * 4);
  p->off_dbpart = align_up(p->off_part + (long long)p->splitk * p->N * p->GR * p->D * p->D * 4);
  p->ws_bwd = align_up(p->off_dbpart + (long long)p->ngroups * p->GT * p->BS * p->D * 4);
  // last, for the LDS-DMA dR GEMM only: 16-bit copies of an FP32 initial hidden
  // state and of the GRU's FP32 candidate-gate cotangents
  p->dma_gemm = gemm_uses_dma(*p) ? 1 : 0;
  p->ws_bwd += s0_copy_bytes(*p) + cand_copy_bytes(*p);
  if (2 * p->xwords_bwd * (p->rs ? 4 : wsz) > 0x7fffffffLL) return FRNN_E_UNSUPPORTED;  // buffer-descriptor range
  return FRNN_OK;
}

int launch(const void* fn, int grid, int block, size_t lds, void* arg, hipStream_t stream) {
  void* args[] = {arg};
  if (hipLaunchKernel(fn, dim3(grid), dim3(block), args, lds, stream) != hipSuccess) {
    (void)hipGetLastError();  // do not leave the error to the caller's next HIP call
    return FRNN_E_LAUNCH;
  }
  return FRNN_OK;
}

// Dynamic LDS beyond the default 64 KiB needs an explicit per-kernel limit.
int set_lds_limit(const void* fn, size_t lds) {
  if (lds > 160 * 1024) return FRNN_E_UNSUPPORTED;
  if (lds <= 64 * 1024) return FRNN_OK;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
    (void)hipGetLastError();
    return FRNN_E_LAUNCH;
  }
  return FRNN_OK;
}

// Workgroups of the kernel one CU holds at once (0 on error).
int blocks_per_cu(const void* fn, int block, size_t lds) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, block, lds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return per_cu;
}

// The persistent kernels need every workgroup of a group resident at once
// (groups never wait on each other). Return in *per_launch how many groups one
// launch may hold: what the GPU holds placement-free, or with every group on
// one XCD, eight times what the busiest XCD holds.
int groups_per_launch(const Plan& p, const void* fn, int block, size_t lds, int* per_launch) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return FRNN_E_LAUNCH;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return FRNN_E_LAUNCH;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, block, lds) != hipSuccess) {
    (void)hipGetLastError();
    return FRNN_E_LAUNCH;
  }
  long long g;
  if (p.flags & FRNN_XCD_SHARED)
    g = (long long)cus * per_cu / p.wpg;
  else
    g = (long long)frnn::kXcds *
        ((long long)(cus / frnn::kXcds) * per_cu /
         (p.wpg + ((p.flags & frnn::kFlagScout) ? std::max(1, p.nscout) : 0)));
  if (g < 1) return FRNN_E_UNSUPPORTED;
  *per_launch = (int)std::min<long long>(g, p.ngroups);
  return FRNN_OK;
}

// Scouts (L2 prefetch of the I/O waves' inputs, one workgroup per group) where
// they cost no extra launch and have a CU to themselves, with the XCD-local
// exchange and a recurrent exchange to pace them by. One workgroup per CU is
// forced, where needed, by asking for more dynamic LDS than half a CU holds: a
// scout's HBM loads would otherwise hold up the polls of a member on its CU
// (and two members on one CU hold up each other's). Sets kFlagScout in the
// launch plan *ap, the groups per launch and the dynamic LDS of the launch.
// Up to `nscout` scouts per group share its touches (fewer where more would
// take another launch).
void use_scouts(const Plan& p, const void* fn, int block, size_t* lds, Plan* ap, int* per_launch, int nscout = 1) {
  if ((p.flags & (FRNN_XCD_SHARED | FRNN_GRAD_CUT)) || g_no_scout.load()) return;
  constexpr size_t kHalfCu = 80 * 1024;
  const size_t lds1 = *lds > kHalfCu ? *lds : kHalfCu + 1024;
  if (set_lds_limit(fn, lds1) != FRNN_OK || blocks_per_cu(fn, block, lds1) != 1) return;
  for (int nsc = std::max(1, nscout); nsc >= 1; --nsc) {
    Plan ps = p;
    ps.flags |= frnn::kFlagScout;
    ps.nscout = nsc;
    int per_scout = 0;
    if (groups_per_launch(ps, fn, block, lds1, &per_scout) == FRNN_OK &&
        (p.ngroups + per_scout - 1) / per_scout == (p.ngroups + *per_launch - 1) / *per_launch) {
      ap->flags |= frnn::kFlagScout;
      ap->nscout = nsc;
      *per_launch = per_scout;
      *lds = lds1;
      return;
    }
  }
}

// Scouts per group in the backward: one per kScoutLines touch slots of a step
// (a scout's CU keeps only so many lines in flight; one that falls behind its
// pace touches lines the I/O waves have already missed on). FRNN_SCOUT_LINES
// (environment, read per call) overrides the share.
int bwd_scouts(const Plan& p) {
  constexpr int kScoutLines = 512;
  int cap = kScoutLines;
  if (const char* e = std::getenv("FRNN_SCOUT_LINES"))
    if (std::atoi(e) > 0) cap = std::atoi(e);
  const int nst = (p.flags & FRNN_OUT_HIDDEN) ? 1 : p.S;
  const int lines = frnn::bwd_scout_lines(p, nst, std::min(p.BS, p.B), p.dt_out == FRNN_F32 ? 4 : 2,
                                          p.dt_save == FRNN_F32 ? 4 : 2);
  return std::min(8, std::max(1, (lines + cap - 1) / cap));
}

// Launch the persistent kernel over all groups in as few launches as residency
// allows; `ap` is the plan inside the kernel arguments `arg`.
int launch_groups(Plan* ap, const void* fn, int block, size_t lds, void* arg, int per_launch, hipStream_t st) {
  int rc = FRNN_OK;
  for (int g0 = 0; g0 < ap->ngroups && rc == FRNN_OK; g0 += per_launch) {
    set_groups(ap, g0, std::min(per_launch, ap->ngroups - g0));
    rc = launch(fn, ap->grid, block, lds, arg, st);
  }
  set_groups(ap, 0, ap->ngroups);
  return rc;
}

int clear(void* base, long long bytes, hipStream_t stream) {
  uint32_t* p = static_cast<uint32_t*>(base);
  long n = (long)(bytes / 4);
  if (n <= 0) return FRNN_OK;
  int grid = (int)std::min<long>(1024, (n + 255) / 256);
  struct {
    uint32_t* p;
    long n;
  } a{p, n};
  void* args[] = {&a.p, &a.n};
  return hipLaunchKernel(frnn::zero_kernel(), dim3(grid), dim3(256), args, 0, stream) == hipSuccess
             ? FRNN_OK
             : FRNN_E_LAUNCH;
}

// Forward launch on a workspace whose layout the plan gives (exchange and slot
// counters at their offsets from `w`; the status word is `status`, which the
// workspace's first word is for frnn_fwd). Clears the exchange and the counters,
// then launches the persistent kernel(s). Allocates nothing.
// ---- input projection (frnn_fwd_projected): its counters follow the forward
// workspace -- ready[nrt] (column tiles done per row tile), then the tile counter
long long proj_row_tiles(const Plan& p) { return ((long long)p.B * p.T + frnn::kProjRows - 1) / frnn::kProjRows; }
long long proj_ws_bytes(const Plan& p) { return p.ws_fwd + align_up(4 * (proj_row_tiles(p) + 1)); }

// FRNN_PROJ_OVERLAP=0 (environment, read per call): run the projection workers
// in a launch of their own before the forward instead of beside it.
bool proj_overlap_allowed() {
  const char* e = std::getenv("FRNN_PROJ_OVERLAP");
  return !(e && *e == '0');
}

// XCDs whose projection workers leave at once: with the XCD-local exchange,
// group slot s of XCD x holds group s * 8 + x, so the first min(groups, 8) XCDs
// host groups. Where every XCD does (or placement is free), none is skipped.
uint32_t proj_skip_xcds(const Plan& p) {
  if ((p.flags & FRNN_XCD_SHARED) || p.ngroups >= frnn::kXcds) return 0u;
  return (1u << p.ngroups) - 1u;
}

// Projection workgroups that can run beside the recurrence in one launch of
// the gated kernel `fg`: one workgroup per CU (more dynamic LDS than half a CU
// holds, so a worker never shares a CU with a member and the recurrence keeps
// its CUs to itself), every group in the one launch, and the CUs the
// recurrence leaves free. Returns 0 where that does not hold; sets *lds.
int proj_workers(const Plan& p, const void* fg, int block, long long tiles, size_t* lds) {
  constexpr size_t kHalfCu = 80 * 1024;
  const size_t l = *lds > kHalfCu ? *lds : kHalfCu + 1024;
  if (set_lds_limit(fg, l) != FRNN_OK || blocks_per_cu(fg, block, l) != 1) return 0;
  int per_launch = 0;
  if (groups_per_launch(p, fg, block, l, &per_launch) != FRNN_OK || per_launch < p.ngroups) return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const int free_cus = cus - p.grid;
  if (free_cus < frnn::kXcds) return 0;
  *lds = l;
  // With XCDs free of groups (proj_skip_xcds), one worker per CU of the whole
  // GPU: the workers dispatched to an XCD with groups leave at once, and those
  // of a free XCD fill its CUs once the recurrence's unused slots there have
  // left. Otherwise the CUs the recurrence leaves, at most one worker wave per tile.
  if (proj_skip_xcds(p)) return cus / frnn::kXcds * frnn::kXcds;
  // a workgroup per tile where the workgroups compute tiles together, a wave per tile otherwise
  const int per_wg = block / 64 >= 4 ? 1 : block / 64;
  const long long useful = (tiles + per_wg - 1) / per_wg;
  return (int)std::min<long long>(free_cus, useful);
}

int fwd_launch(const Plan& p, const void* wx, const void* R, const void* b, const void* s0, void* states_out,
               void* carry_out, void* save, char* w, uint32_t* status, bool allow_timing, hipStream_t st,
               const frnn::ProjArgs* proj = nullptr) {
  if (!wx || !R || !b || !s0 || !states_out) return FRNN_E_INVALID;
  const bool training = (p.flags & FRNN_TRAINING) != 0;
  if (training && !save) return FRNN_E_INVALID;
  const void* fn =
      frnn::recurrence_kernel(p.cell, p.mma, p.KS, ktw_class((p.kt_fwd + p.KS - 1) / p.KS, p.NDT), p.NDT, true);
  if (!fn) return FRNN_E_UNSUPPORTED;
  int rc;
  const long long xbytes = 2 * p.xwords_fwd * (p.mma == FRNN_MMA_F32 ? 8 : 4);
  // exchange and claims (and the projection's counters)
  if ((rc = clear(w + p.off_x, (proj ? proj_ws_bytes(p) : p.ws_fwd) - p.off_x, st)) != FRNN_OK) return rc;
  frnn::FwdArgs a{};
  a.p = p;
  a.wx = wx;
  a.R = R;
  a.bias = b;
  a.s0 = s0;
  a.states = states_out;
  a.carry = carry_out;
  a.save = training ? save : nullptr;
  a.xbuf = w + p.off_x;
  a.xbytes = xbytes;
  a.claim = reinterpret_cast<uint32_t*>(w + p.off_claim_f);
  a.status = status;
  a.spin_limit = g_spin_limit.load();
  a.prof = g_phase_prof.load();
  size_t lds = (size_t)p.NDT * frnn::recurrence_lds_floats(p.cell, true, p.KS) * sizeof(float);
  const int block = 64 * p.NDT * (p.KS + 1);
  int per_launch = 0;
  if ((rc = set_lds_limit(fn, lds)) != FRNN_OK) return rc;
  if ((rc = groups_per_launch(p, fn, block, lds, &per_launch)) != FRNN_OK) return rc;
  if (proj) {
    const long long tiles = (long long)proj->nrt * proj->nct;
    const void* fg = proj_overlap_allowed()
        ? frnn::recurrence_kernel(p.cell, p.mma, p.KS, ktw_class((p.kt_fwd + p.KS - 1) / p.KS, p.NDT), p.NDT, true, true)
        : nullptr;
    size_t lds_g = lds;
    const int nproj = fg ? proj_workers(p, fg, block, tiles, &lds_g) : 0;
    hipEvent_t t0;
    const bool timed = allow_timing && timing_begin(st, &t0);
    if (nproj > 0) {  // one launch: the recurrence's workgroups first, then the projection's
      a.proj = *proj;
      a.proj.skip_xcds = proj_skip_xcds(p);
      // plain (L2-cached) Wx loads, and with them the scouts' L2 prefetch, where
      // no XCD both writes and reads Wx and every Wx row is whole 128-byte lines
      a.proj.plain = a.proj.skip_xcds && proj->ncols % 64 == 0 && (reinterpret_cast<uintptr_t>(proj->wx) & 127) == 0;
      int per_scout = p.ngroups;
      if (a.proj.plain) use_scouts(p, fg, block, &lds_g, &a.p, &per_scout);
      if (per_scout < p.ngroups) return FRNN_E_UNSUPPORTED;  // not reached: the scouts keep one launch
      set_groups(&a.p, 0, p.ngroups);                        // the grid with the scouts' workgroups
      rc = launch(fg, a.p.grid + nproj, block, lds_g, &a, st);
      if (timed) timing_end(0, t0, st);
      return rc;
    }
    // a launch of the projection workers alone, then the forward
    frnn::ProjArgs pa = *proj;
    const void* pk = frnn::proj_kernel(p.mma);
    if ((rc = set_lds_limit(pk, frnn::proj_lds_bytes())) != FRNN_OK) return rc;
    rc = launch(pk, (int)std::min<long long>(4096, tiles), 256, frnn::proj_lds_bytes(), &pa, st);
    if (rc != FRNN_OK) return rc;
    use_scouts(p, fn, block, &lds, &a.p, &per_launch);
    rc = launch_groups(&a.p, fn, block, lds, &a, per_launch, st);
    if (timed) timing_end(0, t0, st);
    return rc;
  }
  use_scouts(p, fn, block, &lds, &a.p, &per_launch);
  hipEvent_t t0;
  const bool timed = allow_timing && timing_begin(st, &t0);
  rc = launch_groups(&a.p, fn, block, lds, &a, per_launch, st);
  if (timed) timing_end(0, t0, st);
  return rc;
}

// ---- scratch of the allocation-free forward (frnn_fwd_noalloc)
// The forward workspace of a problem (status word aside: the caller passes it)
// lives in this file-scope device array, one copy per GPU, held until the
// process ends. Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the symbol): it takes each device's address
// once, with that device current, from hipGetSymbolAddress, and uses that.
constexpr long long kScratchBytes = 8LL << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices] = {};

int scratch_base(char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return FRNN_E_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) return FRNN_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return FRNN_E_LAUNCH;
    }
    g_scratch_ptr[dev] = static_cast<char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return FRNN_OK;
}

}  // namespace

extern "C" {

int frnn_cell_sizes(int cell, int32_t* g_r, int32_t* g_w, int32_t* g_t, int32_t* s) {
  int a, b, c, e;
  if (!cell_sizes(cell, &a, &b, &c, &e)) return FRNN_E_INVALID;
  if (g_r) *g_r = a;
  if (g_w) *g_w = b;
  if (g_t) *g_t = c;
  if (s) *s = e;
  return FRNN_OK;
}

size_t frnn_workspace_bytes(const frnn_desc* d, int which) {
  Plan p;
  if (make_plan(d, &p) != FRNN_OK) return 0;
  switch (which) {
    case 0: return (size_t)p.ws_fwd;
    case 1: return (size_t)p.ws_bwd;
    case 2: return (size_t)p.save_bytes;
    case 3: return (size_t)proj_ws_bytes(p);
  }
  return 0;
}

int frnn_fwd(const frnn_desc* d, const void* wx, const void* R, const void* b, const void* s0,
             void* states_out, void* carry_out, void* save, void* ws, size_t ws_bytes,
             frnn_stream_t stream) {
  Plan p;
  int rc = make_plan(d, &p);
  if (rc != FRNN_OK) return rc;
  if (!ws) return FRNN_E_INVALID;
  if ((long long)ws_bytes < p.ws_fwd) return FRNN_E_WORKSPACE;
  return fwd_launch(p, wx, R, b, s0, states_out, carry_out, save, static_cast<char*>(ws),
                    static_cast<uint32_t*>(ws), true, reinterpret_cast<hipStream_t>(stream));
}

int frnn_fwd_projected(const frnn_desc* d, int32_t input_size, const void* x, const void* w_in, void* wx_out,
                       const void* R, const void* b, const void* s0, void* states_out, void* carry_out, void* save,
                       void* ws, size_t ws_bytes, frnn_stream_t stream) {
  Plan p;
  int rc = make_plan(d, &p);
  if (rc != FRNN_OK) return rc;
  if (!x || !w_in || !wx_out || !ws) return FRNN_E_INVALID;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_in) | reinterpret_cast<uintptr_t>(wx_out)) & 15)
    return FRNN_E_INVALID;  // 16-byte operand runs
  if (input_size < 8 || input_size % 8 != 0) return FRNN_E_UNSUPPORTED;
  if (mma_h16(p.mma) < 0 || p.dt_io != mma_h16(p.mma)) return FRNN_E_UNSUPPORTED;  // 16-bit operands in the MMA type
  if (p.t0 != 0 || p.Ttot != p.T) return FRNN_E_UNSUPPORTED;                       // whole sequences
  if ((long long)ws_bytes < proj_ws_bytes(p)) return FRNN_E_WORKSPACE;
  char* w = static_cast<char*>(ws);
  frnn::ProjArgs pa;
  pa.x = x;
  pa.w = w_in;
  pa.wx = wx_out;
  pa.I = input_size;
  pa.ncols = p.GW * p.N * p.D;
  pa.B = p.B;
  pa.T = p.T;
  pa.nrt = (int)proj_row_tiles(p);
  pa.nct = (pa.ncols + frnn::kProjCols - 1) / frnn::kProjCols;
  pa.ready = reinterpret_cast<uint32_t*>(w + p.ws_fwd);
  pa.next = pa.ready + pa.nrt;
  return fwd_launch(p, wx_out, R, b, s0, states_out, carry_out, save, w, reinterpret_cast<uint32_t*>(w), true,
                    reinterpret_cast<hipStream_t>(stream), &pa);
}

int frnn_fwd_noalloc(const frnn_desc* d, const void* wx, const void* R, const void* b, const void* s0,
                     void* states_out, void* carry_out, void* save, void* status, frnn_stream_t stream) {
  Plan p;
  int rc = make_plan(d, &p);
  if (rc != FRNN_OK) return rc;
  if (!status) return FRNN_E_INVALID;
  if (p.ws_fwd > kScratchBytes) return FRNN_E_SCRATCH;
  char* base = nullptr;
  if ((rc = scratch_base(&base)) != FRNN_OK) return rc;
  return fwd_launch(p, wx, R, b, s0, states_out, carry_out, save, base, static_cast<uint32_t*>(status), false,
                    reinterpret_cast<hipStream_t>(stream));
}

int frnn_bwd(const frnn_desc* d, const void* R, const void* s0, const void* states, const void* save,
             const void* d_states, const void* d_carry, void* dwx, void* dR, void* db, void* ds0, void* ws,
             size_t ws_bytes, frnn_stream_t stream) {
  Plan p;
  int rc = make_plan(d, &p);
  if (rc != FRNN_OK) return rc;
  if (!R || !s0 || !states || !save || !dwx || !dR || !db || !ds0 || !ws) return FRNN_E_INVALID;
  if ((p.flags & FRNN_OUT_LAST) || p.Ttot != p.T || p.t0 != 0) return FRNN_E_INVALID;  // forward-only options
  if ((long long)ws_bytes < p.ws_bwd) return FRNN_E_WORKSPACE;
  const void* fn = p.rs ? frnn::rs_kernel(p.cell, p.mma, p.NDT, p.KSB, p.ptm)
                        : frnn::recurrence_kernel(p.cell, p.mma, p.KSB,
                                                  ktw_class((p.kt_fwd + p.KSB - 1) / p.KSB, p.NDT), p.NDT, false);
  if (!fn) return FRNN_E_UNSUPPORTED;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* w = static_cast<char*>(ws);
  const long long xbytes = 2 * p.xwords_bwd * (p.rs ? 4 : (p.mma == FRNN_MMA_F32 ? 8 : 4));
  if ((rc = clear(w + p.off_x, p.off_dcand - p.off_x, st)) != FRNN_OK) return rc;  // exchange and claims
  frnn::BwdArgs a;
  a.p = p;
  a.R = R;
  a.save = save;
  a.s0 = s0;
  a.d_states = d_states;
  a.d_carry = d_carry;
  a.dwx = dwx;
  a.ds0 = ds0;
  a.dcand = reinterpret_cast<float*>(w + p.off_dcand);
  a.dbpart = reinterpret_cast<float*>(w + p.off_dbpart);
  a.xbuf = w + p.off_x;
  a.xbytes = xbytes;
  a.claim = reinterpret_cast<uint32_t*>(w + p.off_claim_b);
  a.status = reinterpret_cast<uint32_t*>(w);
  a.spin_limit = g_spin_limit.load();
  a.prof = g_phase_prof.load();
  size_t lds = (p.rs ? (size_t)frnn::rs_lds_floats(p.cell, p.NDT)
                     : (size_t)p.NDT * frnn::recurrence_lds_floats(p.cell, false, p.KSB)) * sizeof(float);
  const int block = 64 * p.NDT * (p.KSB + 1);
  int per_launch = 0;
  if ((rc = set_lds_limit(fn, lds)) != FRNN_OK) return rc;
  if ((rc = groups_per_launch(p, fn, block, lds, &per_launch)) != FRNN_OK) return rc;
  use_scouts(p, fn, block, &lds, &a.p, &per_launch, bwd_scouts(p));
  hipEvent_t t0;
  bool timed = timing_begin(st, &t0);
  rc = launch_groups(&a.p, fn, block, lds, &a, per_launch, st);
  if (timed) timing_end(1, t0, st);
  if (rc != FRNN_OK) return rc;

  frnn::GemmArgs g;
  g.p = p;
  g.dwx = dwx;
  g.dcand = a.dcand;
  g.states = states;
  g.s0 = s0;
  g.part = reinterpret_cast<float*>(w + p.off_part);
  g.dbpart = a.dbpart;
  g.zero = w + p.off_claim_b + 2LL * p.ngroups * frnn::kXcds * 4;
  g.dR = dR;
  g.db = db;
  const bool wide = p.D % 64 == 0;
  const int tile = wide ? 64 : 32;
  const long long gwg = (long long)p.N * (p.GR * p.D / tile) * (p.D / tile) * p.splitk;
  timed = timing_begin(st, &t0);
  const int h16 = mma_h16(p.mma);
  // fixed by the plan (the workspace was sized for it), not by the switch's current value
  const bool dma = p.dma_gemm != 0;
  // FP32 -> MMA-type copy (rounded as the register-staged GEMM rounds its operands)
  auto to16 = [&](const float* src, unsigned short* dst, long n16) {
    int dt = h16;
    void* cargs[] = {&src, &dst, &n16, &dt};
    return hipLaunchKernel(frnn::to16_kernel(), dim3((unsigned)std::min<long>(2048, (n16 + 255) / 256)), dim3(256), cargs,
                           0, st) == hipSuccess;
  };
  char* copies = w + p.ws_bwd - s0_copy_bytes(p) - cand_copy_bytes(p);
  if (dma && p.dt_state == FRNN_F32) {
    // the GEMM's h_{-1} rows: s0[0] in the MMA type
    unsigned short* s0h = reinterpret_cast<unsigned short*>(copies + cand_copy_bytes(p));
    if (!to16(static_cast<const float*>(s0), s0h, (long)p.B * p.N * p.D)) return FRNN_E_LAUNCH;
    g.s0 = s0h;
  }
  g.dcand16 = nullptr;
  if (dma && p.cell == FRNN_GRU) {
    // the candidate gate's A rows: its FP32 cotangents in the MMA type
    unsigned short* ch = reinterpret_cast<unsigned short*>(copies);
    if (!to16(a.dcand, ch, (long)p.B * p.T * p.N * p.D)) return FRNN_E_LAUNCH;
    g.dcand16 = ch;
  }
  rc = launch(dma ? frnn::gemm_dma_kernel(p.mma) : frnn::gemm_kernel(p.mma, wide), (int)gwg, wide ? 256 : 64, 0, &g, st);
  const long long nout = (long long)p.N * p.GR * p.D * p.D + (long long)p.GT * p.N * p.D;
  const int rgrid = (int)std::min<long long>(4096, (nout + 255) / 256);
  if (rc == FRNN_OK) rc = launch(frnn::reduce_kernel(), rgrid, 256, 0, &g, st);
  if (timed) timing_end(2, t0, st);
  return rc;
}

int frnn_status(const void* ws, frnn_stream_t stream) {
  if (!ws) return FRNN_E_INVALID;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (hipStreamSynchronize(st) != hipSuccess) return FRNN_E_LAUNCH;
  uint32_t v = 0;
  if (hipMemcpy(&v, ws, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) return FRNN_E_LAUNCH;
  return v == 0 ? FRNN_OK : -(int)v;
}

// Test hook (declared in frnn_plan.h, not part of the public ABI): the launch
// plan of a problem, for the host bounds check of the kernels' addressing.
int frnn_test_plan(const frnn_desc* d, void* plan_out, size_t bytes) {
  if (!plan_out || bytes != sizeof(Plan)) return FRNN_E_INVALID;
  Plan p;
  const int rc = make_plan(d, &p);
  if (rc == FRNN_OK) std::memcpy(plan_out, &p, sizeof(Plan));
  return rc;
}

const char* frnn_strerror(int code) {
  switch (code) {
    case FRNN_OK: return "ok";
    case FRNN_E_INVALID: return "invalid argument (null pointer, unknown enum or non-positive size)";
    case FRNN_E_UNSUPPORTED: return "unsupported configuration (width, register or co-residency limits)";
    case FRNN_E_WORKSPACE: return "workspace smaller than frnn_workspace_bytes()";
    case FRNN_E_LAUNCH: return "HIP kernel launch failed (co-residency or resources)";
    case FRNN_E_TIMEOUT: return "recurrence exchange timed out on the device";
    case FRNN_E_PLACEMENT: return "an XCD received more workgroups than its slots; retry with FRNN_XCD_SHARED";
    case FRNN_E_SCRATCH:
      return "frnn_fwd_noalloc: the problem's forward workspace exceeds the static scratch (8 MiB); use frnn_fwd";
  }
  return "unknown frnn error";
}

void frnn_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  g_timing.on = on != 0;
}

int frnn_timing_read(double* ms3, int32_t* counts3) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  for (int k = 0; k < 3; ++k) {
    if (ms3) ms3[k] = 0.0;
    if (counts3) counts3[k] = 0;
  }
  int rc = FRNN_OK;
  for (auto& r : g_timing.pending) {
    float ms = 0.f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) rc = FRNN_E_LAUNCH;
    if (ms3) ms3[r.kind] += ms;
    if (counts3) counts3[r.kind] += 1;
    g_timing.free_events.push_back(r.a);
    g_timing.free_events.push_back(r.b);
  }
  g_timing.pending.clear();
  return rc;
}

void frnn_set_phase_profile(void* device_words) {
  g_phase_prof.store(static_cast<unsigned long long*>(device_words));
}

void frnn_set_spin_limit(uint32_t polls) { g_spin_limit.store(polls ? polls : kDefaultSpinLimit); }

void frnn_set_scouts(int enable) { g_no_scout.store(enable == 0); }

void frnn_set_gemm_dma(int enable) { g_no_gemm_dma.store(enable == 0); }

}  // extern "C"

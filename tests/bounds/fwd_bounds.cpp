// Host bounds check of the forward recurrence's addressing (CPU only).
//
// For a problem (and, with a step window, each window of a chunked run), it
// enumerates every global element and exchange word the forward kernel's
// workgroups touch -- I/O-wave Wx DMA loads and state / saved-value stores,
// the owners' initial-state loads, bias loads, carry stores and exchange
// stores, the compute waves' resident-R loads and exchange polls, the scouts'
// Wx touches and the slot counters -- using the index functions of
// flashrnn_amd/csrc/frnn_plan.h that the kernels themselves call, with the
// plan that libfrnn.so's make_plan builds (frnn_test_plan), and checks each
// against its buffer's extent. The lane -> work mapping mirrors the kernels
// (fwd_io, fwd_kernel, fwd_scout in frnn_recurrence.h).
//
// Usage: fwd_bounds cell B T N D io(0=f32,1=bf16) flags total_steps windows
// Prints one line per window and "violations N"; exit status 1 on any violation.
#include <cstdio>
#include <cstdlib>

#include "../../flashrnn_amd/csrc/frnn_plan.h"
#include "../../include/frnn.h"

using namespace frnn;

static long long violations = 0;
static void check(const char* what, long long lo, long long hi, long long extent) {
  if (lo < 0 || hi > extent || lo > hi) {
    if (violations < 10)
      std::printf("  VIOLATION %s: [%lld, %lld) outside [0, %lld)\n", what, lo, hi, extent);
    ++violations;
  }
}

static const int kGates[4][4] = {{4, 4, 4, 2}, {3, 3, 4, 1}, {1, 1, 1, 1}, {4, 4, 4, 4}};  // GR GW GT S

static int run_window(const frnn_desc& d) {
  Plan p;
  const int rc = frnn_test_plan(&d, &p, sizeof(p));
  if (rc != FRNN_OK) {
    std::printf("plan rejected: %d\n", rc);
    return rc;
  }
  const int GR = kGates[d.cell][0], GW = kGates[d.cell][1], GT = kGates[d.cell][2], S = kGates[d.cell][3];
  const int B = p.B, T = p.T, N = p.N, D = p.D, TT = p.Ttot;
  const int esz = p.dt_io == FRNN_F32 ? 4 : 2;                // Wx, R, b, states
  const int wp = p.mma == FRNN_MMA_F32 ? 2 : 4;               // exchange words per 16-byte chunk
  const int wsz = p.mma == FRNN_MMA_F32 ? 8 : 4;              // exchange word bytes
  const bool training = (p.flags & FRNN_TRAINING) != 0;
  const int mode = (p.flags & FRNN_OUT_LAST) ? 2 : ((p.flags & FRNN_OUT_HIDDEN) ? 1 : 0);
  const int nst = mode == 0 ? S : 1;
  const int NE = 256 * p.NB;
  // buffer extents (elements, or words for the exchange)
  const long long wx_ext = (long long)B * TT * GW * N * D;
  const long long st_ext = mode == 2 ? (long long)B * N * D : (long long)nst * B * TT * N * D;
  const long long s0_ext = (long long)S * B * N * D;
  const long long b_ext = (long long)GT * N * D, r_ext = (long long)GR * N * D * D;
  const long long sv_ext = training ? p.save_floats : 0;
  const long long x_ext = 2 * p.xwords_fwd;                  // both parities
  const long long claim_ext = 2LL * p.ngroups * kXcds;       // members' and scouts' counters
  if ((long long)p.off_x + x_ext * wsz > p.ws_fwd || p.off_claim_f + claim_ext * 4 > p.ws_fwd)
    check("workspace layout", 0, p.ws_fwd + 1, p.ws_fwd);
  long long touched = 0;

  for (int group = 0; group < p.ngroups; ++group) {
    const int n = group / p.nslab, slab = group % p.nslab;
    const int xgrp = group * p.BS * D;
    const int xpar = p.ngroups * p.BS * D;
    for (int member = 0; member < p.wpg; ++member) {
      for (int team = 0; team < p.NDT; ++team) {
        const int dt = member * p.NDT + team, wgi = group * p.wpg + member;
        // ---- I/O wave
        for (int lane = 0; lane < 64; ++lane) {
          const int e0 = io_elem(lane, 0);
          const ElemPos el = elem_pos(p, slab, dt, e0);
          for (int u = 0; u < T; ++u) {
            for (int g = 0; g < GW; ++g) {
              bool valid;
              const long i = wx_dma_index(p, slab, n, dt, lane, u, g, esz, &valid);
              if (valid) check("Wx DMA", i, i + 16 / esz, wx_ext), ++touched;
            }
            if (!el.real) continue;
            if (mode == 2) {
              if (p.t0 + u == TT - 1) check("last state", last_index(p, el.b, n, el.d), last_index(p, el.b, n, el.d) + 4, st_ext);
            } else {
              for (int k = 0; k < nst; ++k) {
                const long i = state_index(p, k, el.b, u, n, el.d);
                check("state store", i, i + 4, st_ext), ++touched;
              }
            }
            if (training)
              for (int v = 0; v < p.nsave; ++v) {
                const long i = save_index(p, NE, u, wgi, v, team, e0);
                check("save store", i, i + 4, sv_ext);
              }
          }
        }
        // ---- compute waves: owned elements, resident R, exchange
        const int KT = p.kt_fwd;
        for (int kw = 0; kw < p.KS; ++kw) {
          const int kt0 = (kw * KT) / p.KS, nkt = ((kw + 1) * KT) / p.KS - kt0;
          for (int lane = 0; lane < 64; ++lane) {
            const int row = lane & 15, kq = lane >> 4;
            for (int g = 0; g < GR; ++g)
              for (int j = 0; j < nkt; ++j) {
                const long base = (((long)g * N + n) * D + dt * 16 + row) * D + (kt0 + j) * 32 + 8 * kq;
                check("R load", base, base + 8, r_ext);
              }
            // polls: every 16-byte chunk of each run, both parities
            const int cstride_words = 16 * p.BS / wsz;  // the kernels' 16 * BS bytes between a run's chunks
            for (int j = 0; j < nkt; ++j)
              for (int par = 0; par < 2; ++par) {
                const long w = (long)par * xpar + xgrp + xword_rt(wp, p.BS, row, (kt0 + j) * 32 + 8 * kq);
                for (int q = 0; q < 8 / wp; ++q) check("exchange poll", w + q * cstride_words, w + q * cstride_words + wp, x_ext);
                const long wpair = (long)par * xpar + xgrp + xword_rt(wp, p.BS, lane & 7, (kt0 + j) * 32 + 8 * kq);
                for (int q = 0; q < 8 / wp; ++q)
                  check("exchange pair poll", wpair + q * cstride_words, wpair + q * cstride_words + wp, x_ext);
              }
            const int epl = (4 * p.NB + p.KS - 1) / p.KS;
            for (int s = 0; s < epl; ++s) {
              const int oe = s * p.KS * 64 + kw * 64 + lane;
              if (oe >= NE) continue;
              const ElemPos el = elem_pos(p, slab, dt, oe);
              for (int g = 0; g < GT; ++g) check("bias", ((long)g * N + n) * D + el.d, ((long)g * N + n) * D + el.d + 1, b_ext);
              if (!el.real) continue;
              for (int k = 0; k < S; ++k) {
                const long i = carry_index(p, k, el.b, n, el.d);
                check("s0 / carry", i, i + 1, s0_ext);
              }
              for (int par = 0; par < 2; ++par) {
                const long w = (long)par * xpar + xgrp + xword_rt(wp, p.BS, el.bl, el.d);
                check("exchange store", w, w + 1, x_ext);
              }
            }
          }
        }
      }
    }
    // ---- the group's scout (XCD-local launches)
    const int nreal = p.BS < B - slab * p.BS ? p.BS : B - slab * p.BS;
    const int row_bytes = D * esz, lpr = (row_bytes + 127) / 128 + 1;
    for (int u = 0; u < T; ++u)
      for (int r = 0; r < nreal; ++r)
        for (int g = 0; g < GW; ++g)
          for (int l = 0; l < lpr; ++l) {
            const long byte = scout_wx_byte(p, slab, n, r, u, g, l, esz);
            check("scout Wx touch", byte, byte + 4, wx_ext * esz);
          }
    // the scout's pace word: (row 0, k 0) of the group's table, both parities
    for (int par = 0; par < 2; ++par) check("scout pace word", (long)par * xpar + xgrp, (long)par * xpar + xgrp + 1, x_ext);
  }
  // slot counters: members claim claim[g0 * 8 + xcd], scouts claim[(ngroups + g0) * 8 + xcd]
  for (int g0 = 0; g0 < p.ngroups; ++g0)
    for (int xcd = 0; xcd < kXcds; ++xcd) {
      check("member claim", (long)g0 * kXcds + xcd, (long)g0 * kXcds + xcd + 1, claim_ext);
      check("scout claim", ((long)p.ngroups + g0) * kXcds + xcd, ((long)p.ngroups + g0) * kXcds + xcd + 1, claim_ext);
    }
  std::printf("window t0=%d steps=%d of %d: groups %d, workgroups %d, Wx %lld elements (%.2f GiB), %lld checked\n",
              p.t0, T, TT, p.ngroups, p.nwg, wx_ext, wx_ext * esz / 1073741824.0, touched);
  return FRNN_OK;
}

int main(int argc, char** argv) {
  if (argc != 10) {
    std::fprintf(stderr, "usage: fwd_bounds cell B T N D io flags total_steps windows\n");
    return 2;
  }
  frnn_desc d = {};
  d.cell = std::atoi(argv[1]);
  d.batch = std::atoi(argv[2]);
  const int T = std::atoi(argv[3]);
  d.heads = std::atoi(argv[4]);
  d.width = std::atoi(argv[5]);
  d.dtype_io = std::atoi(argv[6]);
  d.dtype_state = FRNN_F32;
  d.mma = d.dtype_io == FRNN_F32 ? FRNN_MMA_F32 : FRNN_MMA_BF16;
  d.flags = std::atoi(argv[7]);
  const int total = std::atoi(argv[8]), windows = std::atoi(argv[9]);
  if (total <= 0 || windows <= 0 || total % windows) return 2;
  const int len = total / windows;
  for (int w = 0; w < windows; ++w) {
    d.steps = windows == 1 ? T : len;
    d.total_steps = windows == 1 ? 0 : total;
    d.step_base = windows == 1 ? 0 : w * len;
    if (run_window(d) != FRNN_OK) return 2;
  }
  std::printf("violations %lld\n", violations);
  return violations ? 1 : 0;
}

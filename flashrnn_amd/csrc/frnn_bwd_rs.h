// Backward time loop with a reduce-scatter exchange (template; each cell
// instantiates it in its own translation unit).
//
// Reference counterpart (behaviour, not code): the backward cell loop,
// flashrnn/flashrnn/fused/flashrnn_fused_backward.cu:130-625.
//
// Per iteration (step t = T-1-it) a group's workgroups exchange partial sums
// of the hidden state's recurrent cotangent instead of the gate cotangents:
//
//  1. the owners of the workgroup's OL = 16*NDT hidden units run the pointwise
//     backward and put their gate cotangents dG (FP32) into LDS;
//  2. after the workgroup barrier, every compute wave multiplies that local
//     dG (k = (unit, gate) of this workgroup only, GR*OL values) by its
//     resident slice of R^T for a share of ALL D output units p, on MFMA, and
//     publishes the D partial sums P_w[b][p] (tagged FP32 words; an output
//     lane holds 4 consecutive p of one batch row: one 16-byte store);
//  3. the owners of unit p poll the wpg partials of p (one per workgroup) and
//     add them in workgroup order: dh_{t-1}[p][b].
//
// A workgroup thus reads D/OL * ... = wpg words per owned element instead of
// the whole G*D-wide dG of every row (the all-gather of bwd_kernel), and no
// LDS reduction or second barrier follows the poll. The product, the
// split-word numerics (dG enters the MFMA as a BF16/FP16 hi + lo pair, FP32
// with FP32 operands) and everything around the exchange (I/O wave, scouts,
// pointwise, cut/clip, db partials) are those of bwd_kernel.
#pragma once

#include "frnn_recurrence.h"

namespace frnn {

// Shape of the local contraction: k = o_local * GRP + g over the OL units of a
// workgroup (GRP = GR slots per unit: 4 for the LSTM and sLSTM, 3 for the GRU,
// 1 for Elman), padded to 32-wide k-tiles; LDS rows of the dG operand are
// padded by 4 floats so the operand reads are conflict-free.
template <int CELL, int NDT>
struct RsShape {
  static constexpr int GR = CellShape<CELL>::GR;
  static constexpr int OL = 16 * NDT;
  static constexpr int GRP = GR;
  static constexpr int KTL = (OL * GRP + 31) / 32;
  static constexpr int KROW = KTL * 32 + 4;
  // floats of LDS: the dG operand [2][16][KROW], then per team the input ring
  // [3][S+NSAVE][NE] and the output staging [2][4][NE]
  static constexpr long team_floats() {
    return (long)kBwdStage * (CellShape<CELL>::S + Cell<CELL>::NSAVE) * 256 + 2L * 4 * 256;
  }
  static constexpr long floats() { return 2L * 16 * KROW + (long)NDT * team_floats(); }
};

// A group's partial-sum table holds, per parity, D * 16 * wpg 32-bit words:
// [v][w][b][p_local] for consumer workgroup v, producer w, batch row b and the
// consumer's unit p_local. A producer lane writes 4 consecutive words (16
// bytes); an owner's poll instruction reads 64 consecutive words per producer
// (its lanes run along p, then b). (A layout in the MFMA output order, one
// tile's store 1 KB of consecutive bytes, measured slower: GRU B16 T512 D768
// backward 3.37 against 3.32 ms, LSTM B16 T1024 D768 7.21 against 6.72 ms.)

// Split an FP32 operand run of 8 k into BF16 / FP16 hi and lo parts (hi + lo
// = the value to about 16 significant bits; the 16-bit backward's numerics).
template <int MMA>
__device__ __forceinline__ void split8(const f32x4& a, const f32x4& b, Frag<MMA>& hi, Frag<MMA>& lo) {
  const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  if constexpr (MMA == MMA_F16) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    typedef __fp16 fp16x2_t __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const f16x2_t h = __builtin_bit_cast(f16x2_t, (fp16x2_t)__builtin_amdgcn_cvt_pkrtz(v[i], v[i + 1]));
      const f16x2_t l = __builtin_bit_cast(
          f16x2_t, (fp16x2_t)__builtin_amdgcn_cvt_pkrtz(v[i] - (float)h[0], v[i + 1] - (float)h[1]));
      hi.v[i] = h[0];
      hi.v[i + 1] = h[1];
      lo.v[i] = l[0];
      lo.v[i + 1] = l[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = f2u(v[i]);
      frag_bits(hi, i, w >> 16);                                  // truncated to BF16
      frag_set(lo, i, v[i] - u2f(w & 0xffff0000u));               // exact remainder, rounded
    }
  }
}

template <int CELL, int MMA, int NDT, int KSC, int PTM>
__global__ void __launch_bounds__(64 * (KSC + 1) * NDT) bwd_rs_kernel(BwdArgs a) {
  using CS = CellShape<CELL>;
  using RS = RsShape<CELL, NDT>;
  constexpr int GR = CS::GR, GW = CS::GW, GT = CS::GT, S = CS::S;
  constexpr int NB = 1, NE = 256, EPLMAX = (4 * NB + KSC - 1) / KSC, KS = KSC;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NIN = S + NSAVE, NOB = Lds<CELL, NB>::NOB;
  constexpr int OL = RS::OL, GRP = RS::GRP, KTL = RS::KTL, KROW = RS::KROW;
  // 4-byte loads per owned element, one per producing workgroup: a group has
  // wpg = D / (16 NDT) <= PTM * KSC workgroups (a wave's PTM output tiles
  // cover D / 16 over NDT * KSC waves)
  constexpr int MAXQ = PTM * KSC;
  static_assert(MAXQ <= 32, "freshness bits of one word");
  const Plan& p = a.p;
  extern __shared__ float lds[];
  Team tm;
  if (blockIdx.x >= p.grid - scout_blocks(p)) {  // a scout
    if (scout_setup(p, tm, a.claim, lds)) bwd_scout<CELL, MMA, true>(a, tm, lds);
    return;
  }
  if (!team_setup(p, tm, a.claim, a.status, KSC, lds)) return;
  const int D = p.D, B = p.B, N = p.N, T = p.T;
  const bool cut = (p.flags & kFlagCut) != 0;
  const bool v1 = CELL == CELL_SLSTM && (p.flags & kFlagV1Grad) != 0;

  float* dgl = lds;                                             // [2][16][KROW]
  float* iring = lds + 2L * 16 * KROW + (long)tm.team * RS::team_floats();  // [3][NIN][NE]
  float* ost = iring + (long)kBwdStage * NIN * NE;              // [2][NOB][NE]
  if (tm.kw == KS) {
    constexpr int SS = SaveSize<CELL, MMA>::value;
    switch (io_sizes(p.dt_io, p.dt_out)) {
      case 0: bwd_io<CELL, MMA, NB, 2, 2, SS>(a, tm, iring, ost); break;
      case 1: bwd_io<CELL, MMA, NB, 2, 4, SS>(a, tm, iring, ost); break;
      default: bwd_io<CELL, MMA, NB, 4, 4, SS>(a, tm, iring, ost); break;
    }
    return;
  }
  // the dG operand starts zero (slots g >= GR and k beyond GR*OL are never written)
  for (int i = (tm.team * KS + tm.kw) * 64 + tm.lane; i < 2 * 16 * KROW; i += NDT * KS * 64) dgl[i] = 0.f;

  Xchg xc;
  {
    uintptr_t xb = reinterpret_cast<uintptr_t>(a.xbuf);
    asm("" : "+v"(xb));
    xc.base = reinterpret_cast<char*>(xb);
  }
  xc.shared_xcd = (p.flags & 2) ? 1 : 0;
  xc.rsrc = __builtin_amdgcn_make_buffer_rsrc(a.xbuf, 0, (int)a.xbytes, 0x00020000);

  const int wpg = p.wpg;
  const int xgrp = tm.group * D * 16 * wpg;       // this group's table
  const int xpar = p.ngroups * D * 16 * wpg;      // words per parity
  const int obase = tm.member * OL;               // first hidden unit of this workgroup

  // ---- this wave's output tiles and its resident R^T slice:
  // A[jj][j][row = p][k] = R[g, n, obase + o, tau*16 + row], k = o*GRP + g
  const int ncw = NDT * KS, cw = tm.team * KS + tm.kw, ntile = D / 16;
  const int tau0 = (cw * ntile) / ncw, npt = ((cw + 1) * ntile) / ncw - tau0;
  Frag<MMA> A[PTM][KTL];
#pragma unroll
  for (int jj = 0; jj < PTM; ++jj)
#pragma unroll
    for (int j = 0; j < KTL; ++j) {
      A[jj][j].zero();
      if (jj < npt) {
        const int prow = (tau0 + jj) * 16 + tm.row;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int k = j * 32 + 8 * tm.kq + i, o = k / GRP, g = k % GRP;
          if (g < GR && o < OL)
            frag_set(A[jj][j], i, ld_val(a.R, (((long)g * N + tm.n) * D + obase + o) * D + prow, p.dt_io));
        }
      }
    }

  // ---- owned elements (pointwise and the poll of their partial sums)
  int oe[EPLMAX];
  bool own[EPLMAX];
  Elem el[EPLMAX];
  float carry[EPLMAX][S], dhrec[EPLMAX], dbacc[EPLMAX][GT];
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    oe[s] = s * KS * 64 + tm.kw * 64 + tm.lane;
    own[s] = oe[s] < NE;
    el[s] = elem_of(p, tm, oe[s] & (NE - 1));
    el[s].real = el[s].real && own[s];
#pragma unroll
    for (int k = 0; k < S; ++k)
      carry[s][k] = (el[s].real && a.d_carry) ? ld_val(a.d_carry, carry_index(p, k, el[s].b, tm.n, el[s].d), p.dt_state)
                                              : 0.f;
    dhrec[s] = 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) dbacc[s][g] = 0.f;
  }
  // sLSTM: (c, n) of the initial state, the (c_{t-1}, n_{t-1}) of step 0
  float init_cn[EPLMAX][2];
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s)
#pragma unroll
    for (int k = 0; k < 2; ++k)
      init_cn[s][k] = (CELL == CELL_SLSTM && el[s].real)
                          ? ld_val(a.s0, carry_index(p, 1 + k, el[s].b, tm.n, el[s].d), p.dt_state)
                          : 0.f;
  // B operand lanes: column c = lane % 16 is batch row c, or with at most 8 real
  // rows (paired) row c % 8, the hi part in columns 0-7 and the lo part in 8-15
  const bool pair = B <= 8;
  const int ocol = tm.lane & 15;
  const int brow = pair ? (ocol & 7) : ocol;
  const bool lo_col = pair && ocol >= 8;

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0, a.prof != nullptr);
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();  // inputs of iterations 0 and 1 staged; the dG operand cleared
  float in_cur[EPLMAX][NIN], in_next[EPLMAX][NIN];
  auto read_in = [&](int it, float (&dst)[EPLMAX][NIN]) {
    const float* ir = iring + (long)(it % kBwdStage) * NIN * NE;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
#pragma unroll
      for (int k = 0; k < NIN; ++k) dst[s][k] = own[s] ? ir[k * NE + oe[s]] : 0.f;
  };
  read_in(0, in_cur);
  bool abort = false;
  for (int it = 0; it < T; ++it) {
    prof.stamp(it, 0);
    const int par = it & 1;
    float* os = ost + (long)par * NE * NOB;
    float* dg = dgl + (long)par * 16 * KROW;
    // ---- 1. owners: pointwise backward of step t = T-1-it; dG into LDS
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int e = oe[s];
      const float* in = in_cur[s];
      float ds[S];
#pragma unroll
      for (int k = 0; k < S; ++k) ds[k] = carry[s][k] + in[k];
      if (p.flags & kFlagClip) {
        const float rec = carry[s][0] + dhrec[s];
        ds[0] = (it == 0 ? rec : fminf(fmaxf(rec, -p.clip), p.clip)) + in[0];
      } else {
        ds[0] += dhrec[s];
      }
      float sv[NSAVE];
#pragma unroll
      for (int v = 0; v < NSAVE; ++v) sv[v] = in[S + v];
      // sLSTM: c and n of step t-1 from that step's saves (staged for the next
      // iteration before the previous barrier), or the initial state at t = 0
      float prev[2] = {0.f, 0.f};
      if constexpr (CELL == CELL_SLSTM) {
        const float* irn = iring + (long)((it + 1) % kBwdStage) * NIN * NE;
#pragma unroll
        for (int k = 0; k < 2; ++k) prev[k] = it + 1 < T ? irn[(S + 1 + k) * NE + e] : init_cn[s][k];
      }
      float dry[GR], dwx[GW], db[GT], cr[S];
      Cell<CELL>::bwd(ds, sv, prev, dry, dwx, db, cr, v1);
      if (!el[s].real) {
#pragma unroll
        for (int g = 0; g < GR; ++g) dry[g] = 0.f;
#pragma unroll
        for (int g = 0; g < GW; ++g) dwx[g] = 0.f;
#pragma unroll
        for (int k = 0; k < S; ++k) cr[k] = 0.f;
      } else {
#pragma unroll
        for (int g = 0; g < GT; ++g) dbacc[s][g] += db[g];
      }
#pragma unroll
      for (int k = 0; k < S; ++k) carry[s][k] = cr[k];
      // dG of (row bl, unit o) at k = o*GRP + g
      float* drow = dg + el[s].bl * KROW + (tm.team * 16 + (e & 15)) * GRP;
      if constexpr (GRP == 4) {
        f32x4 v4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < GR; ++g) v4[g] = dry[g];
        *reinterpret_cast<f32x4*>(drow) = v4;
      } else {
#pragma unroll
        for (int g = 0; g < GRP; ++g) drow[g] = dry[g];
      }
#pragma unroll
      for (int g = 0; g < GW; ++g) os[g * NE + e] = dwx[g];
      if constexpr (CELL == CELL_GRU) os[3 * NE + e] = dry[0];
    }
    prof.mark(3);
    prof.stamp(it, 1);
    lds_barrier();  // dG of the step in LDS; outputs staged; inputs of it+2 staged
    prof.mark(2);
    prof.stamp(it, 2);

    // ---- 2. partial sums of R^T dG over this workgroup's k, for this wave's output tiles
    if (!cut) {
      // B operand fragments of the KTL local k-tiles (shared by every output tile)
      Frag<MMA> bh[KTL], bl[KTL];
#pragma unroll
      for (int j = 0; j < KTL; ++j) {
        const float* src = dg + brow * KROW + j * 32 + 8 * tm.kq;
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(src), x1 = *reinterpret_cast<const f32x4*>(src + 4);
        if constexpr (MMA == MMA_F32) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            bh[j].v[i] = x0[i];
            bh[j].v[4 + i] = x1[i];
          }
        } else {
          split8<MMA>(x0, x1, bh[j], bl[j]);
          if (pair) bh[j] = frag_sel<MMA>(lo_col, bl[j], bh[j]);
        }
      }
      prof.mark(6);
#pragma unroll
      for (int jj = 0; jj < PTM; ++jj) {
        if (jj < npt) {  // (a predicate, not a break: the loop must unroll to keep A in registers)
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KTL; ++j) {
          acc = mma(A[jj][j], bh[j], acc);
          if constexpr (MMA != MMA_F32)
            if (!pair) acc = mma(A[jj][j], bl[j], acc);
        }
        if constexpr (MMA != MMA_F32)
          if (pair) acc = fold_cols8(acc);
        // lane: rows p = tile*16 + 4*(lane/16) + 0..3, column b = lane % 16 (real rows only)
        const int pg = (tau0 + jj) * 16 + 4 * tm.kq;
        const int v = pg / OL, pl = pg % OL, b = ocol;
        if (tm.slab * p.BS + b < B && (!pair || ocol < 8)) {
          const int word = par * xpar + xgrp + ((v * wpg + tm.member) * 16 + b) * OL + pl;
          typedef uint32_t u4 __attribute__((ext_vector_type(4)));
          const uint32_t tg = step_tag(it);
          const u4 w = {split_word(acc[0], tg), split_word(acc[1], tg), split_word(acc[2], tg), split_word(acc[3], tg)};
          uint32_t* q = reinterpret_cast<uint32_t*>(xc.base) + word;
          if (xc.shared_xcd) {
#pragma unroll
            for (int i = 0; i < 4; ++i) __hip_atomic_store(q + i, w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else {
            __builtin_nontemporal_store(w, gptr(reinterpret_cast<u4*>(q)));
          }
        }
        }
      }
    }
    prof.mark(1);
    prof.stamp(it, 3);

    // ---- 3. owners: poll the wpg partial sums of each owned element, add in order
    auto between = [&]() {
      if (it + 1 < T) read_in(it + 1, in_next);
    };
    if (cut) {
      between();
    } else {
      const uint32_t want = ptag(p, it);
      bool first = true;
      uint32_t spins = 0;
      float sum[EPLMAX];
      // One owned element at a time (registers: up to MAXQ loads in flight). A
      // round re-reads only the partials not yet fresh (a producer's words
      // arrive together, so a load skipped by every lane is not issued): the
      // table is read about once per step instead of once per round, which
      // kept the L2 of the group's XCD busy while producers were still
      // storing. The sum runs over the kept words in producer order.
#pragma unroll
      for (int s = 0; s < EPLMAX; ++s) {
        bool done = !el[s].real;
        sum[s] = 0.f;
        const int pl = tm.team * 16 + (oe[s] & 15);
        const int w0 = par * xpar + xgrp + ((tm.member * wpg) * 16 + el[s].bl) * OL + pl;  // + q * 16 * OL
        uint32_t r[MAXQ];
        uint32_t fresh = done ? ~0u : 0u;  // bit q: partial q holds this step's tag
#pragma unroll
        for (int q = 0; q < MAXQ; ++q) r[q] = 0u;
        while (!abort) {
#pragma unroll
          for (int q = 0; q < MAXQ; ++q)
            if (q < wpg && !((fresh >> q) & 1u))
              r[q] = __builtin_amdgcn_raw_buffer_load_b32(xc.rsrc, (w0 + q * 16 * OL) * 4, 0, 16);
          if (first) {
            between();
            first = false;
          }
#pragma unroll
          for (int q = 0; q < MAXQ; ++q)
            if (q < wpg && (r[q] & 3u) == want) fresh |= 1u << q;
          const uint32_t all = wpg >= 32 ? ~0u : (1u << wpg) - 1u;
          if (!done && (fresh & all) == all) {
            done = true;
            float acc = 0.f;
#pragma unroll
            for (int q = 0; q < MAXQ; ++q)
              if (q < wpg) acc += u2f(r[q] & ~3u);
            sum[s] = acc;
          }
          ++spins;
          if (__all(done)) break;
          if (spins >= a.spin_limit) {
            raise_status(a.status, ST_TIMEOUT);
            abort = true;
          } else if ((spins & 63u) == 0 && load_status(a.status) != 0) {
            abort = true;
          }
        }
      }
      if (first) between();
      prof.add(4, spins);
#pragma unroll
      for (int s = 0; s < EPLMAX; ++s) dhrec[s] = el[s].real ? round_op<MMA>(sum[s]) : 0.f;
    }
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
#pragma unroll
      for (int k = 0; k < NIN; ++k) in_cur[s][k] = in_next[s][k];
    prof.mark(0);
    prof.stamp(it, 4);
  }

  // ---- d(initial state), d(bias) partials
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    if (!own[s]) continue;
    if (el[s].real) {
#pragma unroll
      for (int k = 0; k < S; ++k)
        st_val(a.ds0, carry_index(p, k, el[s].b, tm.n, el[s].d), p.dt_state, carry[s][k] + (k == 0 ? dhrec[s] : 0.f));
    }
#pragma unroll
    for (int g = 0; g < GT; ++g)
      a.dbpart[(((long)tm.group * GT + g) * p.BS + el[s].bl) * D + el[s].d] = el[s].real ? dbacc[s][g] : 0.f;
  }
  prof.acc[5] = T;
  prof.flush(a.prof ? a.prof + 128 : nullptr);
  if (a.prof) prof.flush_trace(a.prof + 256 + 128 * 16 * 64, tm);
}

}  // namespace frnn

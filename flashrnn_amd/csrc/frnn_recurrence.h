// Persistent forward and backward time-loop kernels of the fused recurrence
// (templates; each cell instantiates them in its own translation unit).
//
// Reference counterparts (behaviour, not code):
//   forward loop   flashrnn/flashrnn/fused/flashrnn_fused_forward.cu:147-660
//   backward loop  flashrnn/flashrnn/fused/flashrnn_fused_backward.cu:130-625
#pragma once

#include "frnn_cells.h"
#include "frnn_device.h"
#include "frnn_kernels.h"
#include "frnn_plan.h"

namespace frnn {

// ============================================================== helpers
struct Team {
  int lane, w, row, kq;  // lane in wave, wave in workgroup, lane%16, lane/16
  int team, kw;          // hidden tile of this wave in the workgroup, its contraction split
  int group, member, n, slab;
};

__device__ __forceinline__ long save_index(const Plan& p, int t, int wgi, int v, int s, int w, int lane) {
  const int wpw = p.NDT * p.KS;  // waves per workgroup
  const long per = (long)wpw * 64 * p.epl;
  return (((long)t * p.nwg + wgi) * p.nsave + v) * per + (long)s * wpw * 64 + w * 64 + lane;
}

// dR-GEMM operand copies: BF16 (bf16 path) or FP32 (f32 path), 8 batch rows innermost.
template <int MMA>
__device__ __forceinline__ void gemm_store(void* base, long i, float v) {
  if constexpr (MMA == MMA_BF16) static_cast<unsigned short*>(base)[i] = (unsigned short)bf16_bits(v);
  else static_cast<float*>(base)[i] = v;
}

// Poll the exchange until every 8-word run this wave needs carries `tag`.
// Runs of padded batch rows are not read (their fragments stay zero).
template <int MMA, int NB, int NF>
__device__ __forceinline__ void gather(const Xchg& x, const long (&word)[NB][NF], const bool (&bval)[NB],
                                       int nf, uint32_t tag, Frag<MMA> (&X)[NB][NF], uint32_t* status,
                                       uint32_t spin_limit, bool& abort) {
  if (abort) return;
  uint32_t spins = 0;
  while (true) {
    Run<MMA> r[NB][NF];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int j = 0; j < NF; ++j)
        if (j < nf && bval[bt]) xload<MMA>(x, word[bt][j], r[bt][j]);
    bool ok = true;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int j = 0; j < NF; ++j)
        if (j < nf && bval[bt]) ok &= xunpack<MMA>(r[bt][j], tag, X[bt][j]);
    if (__all(ok)) return;
    ++spins;
    if (spins >= spin_limit) {
      raise_status(status, ST_TIMEOUT);
      abort = true;
      return;
    }
    if ((spins & 63u) == 0 && load_status(status) != 0) {
      abort = true;
      return;
    }
  }
}

// ============================================================== forward
template <int CELL, int MMA, int KTW, int NB>
__global__ void __launch_bounds__(512) fwd_kernel(FwdArgs a) {
  using CS = CellShape<CELL>;
  constexpr int GR = CS::GR, GW = CS::GW, GT = CS::GT, S = CS::S;
  constexpr int EPLMAX = 4 * NB;
  constexpr int NSAVE = Cell<CELL>::NSAVE;
  const Plan& p = a.p;
  Team tm;
  if (!wg_decode(p, blockIdx.x, &tm.group, &tm.member)) return;
  if (!(p.flags & 2) && xcc_id() != (uint32_t)(blockIdx.x % kXcds)) {
    if (threadIdx.x == 0) raise_status(a.status, ST_PLACEMENT);
    return;  // the whole workgroup leaves together; partners time out or see the status
  }
  tm.lane = threadIdx.x & 63;
  tm.w = threadIdx.x >> 6;
  tm.team = tm.w / p.KS;
  tm.kw = tm.w % p.KS;
  tm.row = tm.lane & 15;
  tm.kq = tm.lane >> 4;
  tm.n = tm.group / p.nslab;
  tm.slab = tm.group % p.nslab;
  const int KS = p.KS, D = p.D, B = p.B, T = p.T, N = p.N, dt = tm.member * p.NDT + tm.team;
  const int wgi = tm.group * p.wpg + tm.member;
  const bool training = (p.flags & 1) != 0;

  extern __shared__ float red[];  // [2][NDT][KS][NB][GR][64][4]

  Xchg xc;
  xc.base = a.xbuf;
  xc.shared_xcd = (p.flags & 2) ? 1 : 0;
  xc.rsrc = __builtin_amdgcn_make_buffer_rsrc(a.xbuf, 0, (int)a.xbytes, 0x00020000);

  // ---- contraction split: k-tiles [kt0, kt0 + nkt) of D/32
  const int KT = p.kt_fwd;
  const int kt0 = (tm.kw * KT) / KS;
  const int nkt = ((tm.kw + 1) * KT) / KS - kt0;

  // ---- resident recurrent weights: A[g][j] = R[g, n, dt*16 + row, (kt0+j)*32 + 8*kq + 0..7]
  Frag<MMA> A[GR][KTW];
#pragma unroll
  for (int g = 0; g < GR; ++g)
#pragma unroll
    for (int j = 0; j < KTW; ++j) {
      A[g][j].zero();
      if (j < nkt) {
        const long base = (((long)g * N + tm.n) * D + dt * 16 + tm.row) * D + (kt0 + j) * 32 + 8 * tm.kq;
#pragma unroll
        for (int i = 0; i < 8; ++i) frag_set(A[g][j], i, ld_val(a.R, base + i, p.dt_io));
      }
    }

  // ---- exchange word index of every run this wave reads (h_{t-1}[b][k])
  long xword[NB][KTW];
  bool bval[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int bl = bt * 16 + tm.row;
    bval[bt] = tm.slab * p.BS + bl < B;
#pragma unroll
    for (int j = 0; j < KTW; ++j) xword[bt][j] = ((long)tm.group * p.BS + bl) * D + (kt0 + j) * 32 + 8 * tm.kq;
  }
  const long xpar = (long)p.ngroups * p.BS * D;  // words per parity

  // ---- owned elements (d, b): element e = s*KS*64 + kw*64 + lane of the team's NB*256 tile elements
  int od[EPLMAX], ob[EPLMAX], obl[EPLMAX], osrc[EPLMAX];
  bool own[EPLMAX], real[EPLMAX];
  float st[EPLMAX][S], bias[EPLMAX][GT];
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    const int e = s * KS * 64 + tm.kw * 64 + tm.lane;
    own[s] = s < p.epl && e < NB * 256;
    const int bt = e >> 8, r = e & 255, dd = r & 15, bb = r >> 4;
    od[s] = dt * 16 + dd;
    obl[s] = bt * 16 + bb;
    ob[s] = tm.slab * p.BS + obl[s];
    real[s] = own[s] && ob[s] < B;
    // partial-sum source in the MFMA output layout: lane (dd/4)*16 + bb, register dd%4, tile bt
    osrc[s] = ((bt * GR) * 64 + (dd >> 2) * 16 + bb) * 4 + (dd & 3);
#pragma unroll
    for (int k = 0; k < S; ++k)
      st[s][k] = real[s] ? ld_val(a.s0, (((long)k * B + ob[s]) * N + tm.n) * D + od[s], p.dt_state) : 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) bias[s][g] = own[s] ? ld_val(a.bias, ((long)g * N + tm.n) * D + od[s], p.dt_io) : 0.f;
  }

  // sLSTM: the reference's global predicate all(n0 == 0) over the whole call's initial state
  uint32_t zflag = 0;
  if constexpr (CELL == CELL_SLSTM) {
    int nz = 0;
    const long cnt = (long)B * N * D;
    for (long i = threadIdx.x; i < cnt; i += blockDim.x) nz |= ld_val(a.s0, 2 * cnt + i, p.dt_state) != 0.f;
    zflag = __syncthreads_or(nz) ? 0u : 1u;
  }

  // ---- dR-GEMM copy of h_{-1} (slot 0)
  const long hs_row = (long)p.Bp8 / 8;
  if (training) {
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
      if (own[s] && ob[s] < p.Bp8)
        gemm_store<MMA>(a.hsave, ((((long)tm.n * p.T) * hs_row + ob[s] / 8) * D + od[s]) * 8 + (ob[s] & 7),
                        real[s] ? st[s][0] : 0.f);
  }

  // ---- Wx prefetch (one step ahead)
  float xw[EPLMAX][GW];
  const long wx_t = (long)GW * N * D;  // stride of t in Wx [B,T,G,N,D]
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s)
#pragma unroll
    for (int g = 0; g < GW; ++g)
      xw[s][g] = real[s] ? ld_val(a.wx, ((long)ob[s] * T) * wx_t + ((long)g * N + tm.n) * D + od[s], p.dt_io) : 0.f;

  Frag<MMA> X[NB][KTW];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt)
#pragma unroll
    for (int j = 0; j < KTW; ++j) X[bt][j].zero();

  bool abort = false;
  for (int t = 0; t < T; ++t) {
    // ---- 1. h_{t-1} fragments
    if (t == 0) {
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int j = 0; j < KTW; ++j)
          if (j < nkt && bval[bt]) {
            const int b = tm.slab * p.BS + bt * 16 + tm.row;
            const long base = ((long)b * N + tm.n) * D + (kt0 + j) * 32 + 8 * tm.kq;
#pragma unroll
            for (int i = 0; i < 8; ++i) frag_set(X[bt][j], i, ld_val(a.s0, base + i, p.dt_state));
          }
    } else {
      long wd[NB][KTW];
      const long off = ((t - 1) & 1) * xpar;
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int j = 0; j < KTW; ++j) wd[bt][j] = xword[bt][j] + off;
      gather<MMA, NB, KTW>(xc, wd, bval, nkt, step_tag(t - 1), X, a.status, a.spin_limit, abort);
    }

    // ---- 2. partial R . h over this wave's k-tiles
    f32x4 acc[NB][GR];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int g = 0; g < GR; ++g) acc[bt][g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KTW; ++j)
      if (j < nkt) {
#pragma unroll
        for (int g = 0; g < GR; ++g)
#pragma unroll
          for (int bt = 0; bt < NB; ++bt) acc[bt][g] = mma(A[g][j], X[bt][j], acc[bt][g]);
      }

    // ---- 3. partials to LDS, one barrier per step (double-buffered by parity)
    float* rp = red + ((long)(t & 1) * p.NDT + tm.team) * KS * NB * GR * 256;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int g = 0; g < GR; ++g)
        *reinterpret_cast<f32x4*>(rp + (((tm.kw * NB + bt) * GR + g) * 64 + tm.lane) * 4) = acc[bt][g];
    __syncthreads();

    // ---- 4. owners: gates, cell, outputs, exchange
    const bool last = t + 1 == T;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      float ry[GR];
#pragma unroll
      for (int g = 0; g < GR; ++g) {
        float v = 0.f;
        for (int w2 = 0; w2 < KS; ++w2) v += rp[w2 * NB * GR * 256 + osrc[s] + g * 256];
        ry[g] = v;
      }
      float xcur[GW];
#pragma unroll
      for (int g = 0; g < GW; ++g) xcur[g] = xw[s][g];
      if (!last) {
#pragma unroll
        for (int g = 0; g < GW; ++g)
          xw[s][g] = real[s] ? ld_val(a.wx, ((long)ob[s] * T + t + 1) * wx_t + ((long)g * N + tm.n) * D + od[s], p.dt_io)
                             : 0.f;
      }
      float sv[NSAVE];
      if constexpr (CELL == CELL_GRU) {
        Cell<CELL_GRU>::fwd3(ry, xcur, bias[s], st[s], sv);
      } else {
        float g4[GR];
#pragma unroll
        for (int g = 0; g < GR; ++g) g4[g] = xcur[g] + ry[g] + bias[s][g];
        Cell<CELL>::fwd(g4, st[s], sv, (CELL == CELL_SLSTM && t == 0) ? zflag : 0u);
      }
      if (real[s]) {
#pragma unroll
        for (int k = 0; k < S; ++k)
          st_val(a.states, ((((long)k * B + ob[s]) * T + t) * N + tm.n) * D + od[s], p.dt_io, st[s][k]);
        if (!last)
          xstore<MMA>(xc, (t & 1) * xpar + ((long)tm.group * p.BS + obl[s]) * D + od[s], st[s][0], step_tag(t));
      }
      if (training) {
#pragma unroll
        for (int v = 0; v < NSAVE; ++v) a.save[save_index(p, t, wgi, v, s, tm.w, tm.lane)] = sv[v];
        if (!last && ob[s] < p.Bp8)
          gemm_store<MMA>(a.hsave, ((((long)tm.n * T + t + 1) * hs_row + ob[s] / 8) * D + od[s]) * 8 + (ob[s] & 7),
                          real[s] ? st[s][0] : 0.f);
      }
    }
  }

  // ---- carry: the last state in full precision
  if (a.carry) {
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
      if (real[s])
#pragma unroll
        for (int k = 0; k < S; ++k)
          st_val(a.carry, (((long)k * B + ob[s]) * N + tm.n) * D + od[s], p.dt_state, st[s][k]);
  }
}

// ============================================================== backward
template <int CELL, int MMA, int KTW, int NB>
__global__ void __launch_bounds__(512) bwd_kernel(BwdArgs a) {
  using CS = CellShape<CELL>;
  constexpr int GR = CS::GR, GW = CS::GW, GT = CS::GT, S = CS::S;
  constexpr int EPLMAX = 4 * NB;
  constexpr int NSAVE = Cell<CELL>::NSAVE;
  constexpr int NF = GR * KTW;  // max fragments of R^T per wave
  const Plan& p = a.p;
  Team tm;
  if (!wg_decode(p, blockIdx.x, &tm.group, &tm.member)) return;
  if (!(p.flags & 2) && xcc_id() != (uint32_t)(blockIdx.x % kXcds)) {
    if (threadIdx.x == 0) raise_status(a.status, ST_PLACEMENT);
    return;
  }
  tm.lane = threadIdx.x & 63;
  tm.w = threadIdx.x >> 6;
  tm.team = tm.w / p.KS;
  tm.kw = tm.w % p.KS;
  tm.row = tm.lane & 15;
  tm.kq = tm.lane >> 4;
  tm.n = tm.group / p.nslab;
  tm.slab = tm.group % p.nslab;
  const int KS = p.KS, D = p.D, B = p.B, T = p.T, N = p.N, dt = tm.member * p.NDT + tm.team;
  const int wgi = tm.group * p.wpg + tm.member;
  const int GD = GR * D;

  extern __shared__ float red[];  // [2][NDT][KS][NB][64][4]

  Xchg xc;
  xc.base = a.xbuf;
  xc.shared_xcd = (p.flags & 2) ? 1 : 0;
  xc.rsrc = __builtin_amdgcn_make_buffer_rsrc(a.xbuf, 0, (int)a.xbytes, 0x00020000);

  // ---- contraction split over the (g, o) k-tiles of dG: [kt0, kt0 + nkt) of GR*D/32
  const int KT = p.kt_bwd;
  const int kt0 = (tm.kw * KT) / KS;
  const int nkt = ((tm.kw + 1) * KT) / KS - kt0;

  // ---- resident R^T: A[j][row = p][k = (g, o)] = R[g, n, o, dt*16 + row]
  Frag<MMA> A[NF];
#pragma unroll
  for (int j = 0; j < NF; ++j) {
    A[j].zero();
    if (j < nkt) {
      const int kk = (kt0 + j) * 32 + 8 * tm.kq;
      const int g = kk / D, o = kk % D;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        frag_set(A[j], i, ld_val(a.R, (((long)g * N + tm.n) * D + o + i) * D + dt * 16 + tm.row, p.dt_io));
    }
  }

  long xword[NB][NF];
  bool bval[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int bl = bt * 16 + tm.row;
    bval[bt] = tm.slab * p.BS + bl < B;
#pragma unroll
    for (int j = 0; j < NF; ++j) xword[bt][j] = ((long)tm.group * p.BS + bl) * GD + (kt0 + j) * 32 + 8 * tm.kq;
  }
  const long xpar = (long)p.ngroups * p.BS * GD;

  int od[EPLMAX], ob[EPLMAX], obl[EPLMAX], osrc[EPLMAX];
  bool own[EPLMAX], real[EPLMAX];
  float carry[EPLMAX][S], dhrec[EPLMAX], dbacc[EPLMAX][GT];
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    const int e = s * KS * 64 + tm.kw * 64 + tm.lane;
    own[s] = s < p.epl && e < NB * 256;
    const int bt = e >> 8, r = e & 255, dd = r & 15, bb = r >> 4;
    od[s] = dt * 16 + dd;
    obl[s] = bt * 16 + bb;
    ob[s] = tm.slab * p.BS + obl[s];
    real[s] = own[s] && ob[s] < B;
    osrc[s] = (bt * 64 + (dd >> 2) * 16 + bb) * 4 + (dd & 3);
#pragma unroll
    for (int k = 0; k < S; ++k)
      carry[s][k] = (real[s] && a.d_carry) ? ld_val(a.d_carry, (((long)k * B + ob[s]) * N + tm.n) * D + od[s], p.dt_state) : 0.f;
    dhrec[s] = 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) dbacc[s][g] = 0.f;
  }

  Frag<MMA> X[NB][NF];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt)
#pragma unroll
    for (int j = 0; j < NF; ++j) X[bt][j].zero();

  const long hs_row = (long)p.Bp8 / 8;
  const long wx_t = (long)GW * N * D;
  bool abort = false;
  for (int it = 0; it < T; ++it) {
    const int t = T - 1 - it;
    const long xoff = (it & 1) * xpar;
    // ---- 1. owners: pointwise backward of step t, publish dG_t
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      float ds[S];
#pragma unroll
      for (int k = 0; k < S; ++k) {
        float v = carry[s][k];
        if (real[s] && a.d_states) v += ld_val(a.d_states, ((((long)k * B + ob[s]) * T + t) * N + tm.n) * D + od[s], p.dt_io);
        ds[k] = v;
      }
      ds[0] += dhrec[s];
      float sv[NSAVE];
#pragma unroll
      for (int v = 0; v < NSAVE; ++v) sv[v] = a.save[save_index(p, t, wgi, v, s, tm.w, tm.lane)];
      float dry[GR], dwx[GW], db[GT], cr[S];
      Cell<CELL>::bwd(ds, sv, dry, dwx, db, cr);
      if (!real[s]) {
#pragma unroll
        for (int g = 0; g < GR; ++g) dry[g] = 0.f;
      }
#pragma unroll
      for (int k = 0; k < S; ++k) carry[s][k] = real[s] ? cr[k] : 0.f;
      if (real[s]) {
#pragma unroll
        for (int g = 0; g < GT; ++g) dbacc[s][g] += db[g];
#pragma unroll
        for (int g = 0; g < GW; ++g)
          st_val(a.dwx, ((long)ob[s] * T + t) * wx_t + ((long)g * N + tm.n) * D + od[s], p.dt_io, dwx[g]);
#pragma unroll
        for (int g = 0; g < GR; ++g)
          xstore<MMA>(xc, xoff + ((long)tm.group * p.BS + obl[s]) * GD + g * D + od[s], dry[g], step_tag(it));
      }
      if (ob[s] < p.Bp8) {
#pragma unroll
        for (int g = 0; g < GR; ++g)
          gemm_store<MMA>(a.dgsave, ((((long)tm.n * T + t) * hs_row + ob[s] / 8) * GD + g * D + od[s]) * 8 + (ob[s] & 7),
                          dry[g]);
      }
    }

    // ---- 2. dh_{t-1} partial = R^T dG_t over this wave's k-tiles
    long wd[NB][NF];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int j = 0; j < NF; ++j) wd[bt][j] = xword[bt][j] + xoff;
    gather<MMA, NB, NF>(xc, wd, bval, nkt, step_tag(it), X, a.status, a.spin_limit, abort);
    f32x4 acc[NB];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) acc[bt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NF; ++j)
      if (j < nkt) {
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) acc[bt] = mma(A[j], X[bt][j], acc[bt]);
      }
    float* rp = red + ((long)(it & 1) * p.NDT + tm.team) * KS * NB * 256;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
      *reinterpret_cast<f32x4*>(rp + ((tm.kw * NB + bt) * 64 + tm.lane) * 4) = acc[bt];
    __syncthreads();

    // ---- 3. owners: reduce -> recurrent cotangent of h_{t-1}
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      float v = 0.f;
      for (int w2 = 0; w2 < KS; ++w2) v += rp[w2 * NB * 256 + osrc[s]];
      // the BF16 policy rounds the cotangent of the rounded hidden operand
      dhrec[s] = real[s] ? (MMA == MMA_BF16 ? round_bf16(v) : v) : 0.f;
    }
  }

  // ---- d(initial state), d(bias) partials
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    if (!own[s]) continue;
    if (real[s]) {
#pragma unroll
      for (int k = 0; k < S; ++k) {
        const float v = carry[s][k] + (k == 0 ? dhrec[s] : 0.f);
        st_val(a.ds0, (((long)k * B + ob[s]) * N + tm.n) * D + od[s], p.dt_state, v);
      }
    }
#pragma unroll
    for (int g = 0; g < GT; ++g)
      a.dbpart[(((long)tm.group * GT + g) * p.BS + obl[s]) * D + od[s]] = real[s] ? dbacc[s][g] : 0.f;
  }
}

}  // namespace frnn

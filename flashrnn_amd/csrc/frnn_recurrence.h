// Persistent forward and backward time-loop kernels of the fused recurrence
// (templates; each cell instantiates them in its own translation unit).
//
// Reference counterparts (behaviour, not code):
//   forward loop   flashrnn/flashrnn/fused/flashrnn_fused_forward.cu:147-660
//   backward loop  flashrnn/flashrnn/fused/flashrnn_fused_backward.cu:130-625
//
// Workgroup = NDT hidden tiles ("teams"); a team is KS compute waves plus one
// I/O wave. The compute waves hold the team's slice of R (forward) or R^T
// (backward) in registers, run the per-step product on MFMA over their share
// of the contraction, reduce through LDS, apply the cell to the elements they
// own and publish the new exchange words. Their only global-memory traffic in
// the time loop is that exchange (L2). The I/O wave streams everything else
// through LDS: the next steps' inputs (Wx forward; saved activations and the
// incoming state cotangents backward) into a ring several steps ahead, and the
// previous step's outputs from a double-buffered staging area to HBM. On gfx9
// one wave's loads and stores retire through a single in-order counter, so
// keeping HBM traffic off the compute waves keeps HBM latency off the
// recurrence's critical path.
//
// Element e of a team (0 <= e < 256*NB) is (batch tile e>>8, hidden unit
// e&15 of the tile, batch row (e>>4)&15). Compute lane (kw, lane) owns the
// elements e = s*KS*64 + kw*64 + lane; I/O lane l serves e = l + 64*i.
#pragma once

#include "frnn_cells.h"
#include "frnn_device.h"
#include "frnn_kernels.h"
#include "frnn_plan.h"

namespace frnn {

constexpr int kFwdRing = 4;  // Wx steps staged ahead

template <int CELL>
struct BwdRing {  // input steps staged ahead, bounded by the I/O wave's registers
  static constexpr int P = 2;
};

template <int CELL, int NB>
struct Lds {
  static constexpr int NE = NB * 256;
  static constexpr int GR = CellShape<CELL>::GR, GW = CellShape<CELL>::GW, S = CellShape<CELL>::S;
  static constexpr int NSAVE = Cell<CELL>::NSAVE;
  // floats per team
  __host__ __device__ static constexpr long fwd(int KS) {
    return 2L * KS * NB * GR * 256 + (long)kFwdRing * GW * NE + 2L * (S + NSAVE) * NE;
  }
  __host__ __device__ static constexpr long bwd(int KS) {
    return 2L * KS * NB * 256 + (long)BwdRing<CELL>::P * (S + NSAVE) * NE + 2L * (GW + (CELL == CELL_GRU ? 1 : 0)) * NE;
  }
};

struct Team {
  int lane, w, row, kq;  // lane in wave, wave in workgroup, lane%16, lane/16
  int team, kw;          // hidden tile (team) of this wave, its contraction split (kw == KS: I/O wave)
  int group, member, n, slab, dt, wgi;
};

__device__ __forceinline__ bool team_setup(const Plan& p, Team& tm, uint32_t* status) {
  if (!wg_decode(p, blockIdx.x, &tm.group, &tm.member)) return false;
  if (!(p.flags & 2) && xcc_id() != (uint32_t)(blockIdx.x % kXcds)) {
    if (threadIdx.x == 0) raise_status(status, ST_PLACEMENT);
    return false;  // the whole workgroup leaves together; partners time out or see the status
  }
  tm.lane = threadIdx.x & 63;
  tm.w = threadIdx.x >> 6;
  tm.team = tm.w / (p.KS + 1);
  tm.kw = tm.w % (p.KS + 1);
  tm.row = tm.lane & 15;
  tm.kq = tm.lane >> 4;
  tm.n = tm.group / p.nslab;
  tm.slab = tm.group % p.nslab;
  tm.dt = tm.member * p.NDT + tm.team;
  tm.wgi = tm.group * p.wpg + tm.member;
  return true;
}

// Element e of the team -> hidden unit d, slab row bl, batch row b.
struct Elem {
  int d, bl, b;
  bool real;
};
__device__ __forceinline__ Elem elem_of(const Plan& p, const Team& tm, int e) {
  Elem x;
  const int bt = e >> 8, r = e & 255;
  x.d = tm.dt * 16 + (r & 15);
  x.bl = bt * 16 + (r >> 4);
  x.b = tm.slab * p.BS + x.bl;
  x.real = x.b < p.B;
  return x;
}
// Partial-sum position of element e in the MFMA output layout of its batch
// tile: lane (dd/4)*16 + row, register dd%4 (dd = hidden unit in the tile).
__device__ __forceinline__ int mfma_pos(int e) {
  const int r = e & 255, dd = r & 15, bb = r >> 4;
  return ((dd >> 2) * 16 + bb) * 4 + (dd & 3);
}

// Lane-native saved values: [t][workgroup][value][team*NE + e].
__device__ __forceinline__ long save_index(const Plan& p, int ne, int t, int wgi, int v, int team, int e) {
  const long per = (long)p.NDT * ne;
  return (((long)t * p.nwg + wgi) * p.nsave + v) * per + (long)team * ne + e;
}

// Phase profile of every wave of workgroup 0 (8 words per wave). Compute
// waves: cycles in [0] exchange wait, [1] MFMA + LDS partials, [2] barrier,
// [3] owners' cell work, [4] exchange polls, [5] steps. I/O waves: [0] ring
// fill (waits for its loads), [1] load issue, [2] barrier, [3] output drain.
struct Prof {
  unsigned long long acc[6];
  unsigned long long t;
  bool on;
  __device__ __forceinline__ void init(bool enable) {
    on = enable;
    for (int i = 0; i < 6; ++i) acc[i] = 0;
    t = on ? clock64() : 0;
  }
  __device__ __forceinline__ void mark(int k) {
    if (!on) return;
    unsigned long long now = clock64();
    acc[k] += now - t;
    t = now;
  }
  __device__ __forceinline__ void add(int k, unsigned long long v) {
    if (on) acc[k] += v;
  }
  __device__ __forceinline__ void flush(unsigned long long* out) {
    if (on && (threadIdx.x & 63) == 0)
      for (int i = 0; i < 6; ++i) out[(threadIdx.x >> 6) * 8 + i] = acc[i];
  }
};

// Poll the exchange until every 8-word run this wave needs carries `tag`.
// Runs of padded batch rows are not read (their fragments stay zero).
// Returns the number of polls.
template <int MMA, int NB, int NF>
__device__ __forceinline__ uint32_t gather(const Xchg& x, const int (&word)[NB][NF], const bool (&bval)[NB],
                                           int off, int nf, uint32_t tag, Frag<MMA> (&X)[NB][NF],
                                           uint32_t* status, uint32_t spin_limit, bool& abort) {
  if (abort) return 0;
  uint32_t spins = 0;
  while (true) {
    Run<MMA> r[NB][NF];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int j = 0; j < NF; ++j)
        if (j < nf && bval[bt]) xload<MMA>(x, word[bt][j] + off, r[bt][j]);
    bool ok = true;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int j = 0; j < NF; ++j)
        if (j < nf && bval[bt]) ok &= xunpack<MMA>(r[bt][j], tag, X[bt][j]);
    ++spins;
    if (__all(ok)) return spins;
    if (spins >= spin_limit) {
      raise_status(status, ST_TIMEOUT);
      abort = true;
      return spins;
    }
    if ((spins & 63u) == 0 && load_status(status) != 0) {
      abort = true;
      return spins;
    }
  }
}

// ====================================================================== forward
// I/O lane l serves the elements e = 256*(i/4) + 4*l + i%4: four consecutive
// hidden units of one batch row, so every global access is one 8/16-byte
// vector access and every LDS access one 16-byte access.
__device__ __forceinline__ int io_elem(int lane, int i) { return 256 * (i >> 2) + 4 * lane + (i & 3); }

// I/O wave of a team: Wx of step t+P into the ring, outputs of step t-1 to HBM.
template <int CELL, int MMA, int NB>
__device__ void fwd_io(const FwdArgs& a, const Team& tm, float* xring, float* ost) {
  using CS = CellShape<CELL>;
  constexpr int GW = CS::GW, S = CS::S, NE = NB * 256, IOQ = NB, P = kFwdRing;  // IOQ quads per lane
  constexpr int NSAVE = Cell<CELL>::NSAVE, NOUT = S + NSAVE;
  const Plan& p = a.p;
  const int T = p.T, N = p.N, D = p.D, B = p.B;
  const bool training = (p.flags & 1) != 0;
  const long wx_t = (long)GW * N * D;
  Elem el[IOQ];
  int e0[IOQ];
#pragma unroll
  for (int q = 0; q < IOQ; ++q) {
    e0[q] = io_elem(tm.lane, 4 * q);
    el[q] = elem_of(p, tm, e0[q]);
  }
  auto load_wx = [&](int t, u32x4 (&dst)[IOQ][GW]) {
#pragma unroll
    for (int q = 0; q < IOQ; ++q)
#pragma unroll
      for (int g = 0; g < GW; ++g)
        dst[q][g] = el[q].real
                        ? ld4_raw(a.wx, ((long)el[q].b * T + t) * wx_t + ((long)g * N + tm.n) * D + el[q].d, p.dt_io)
                        : u32x4{0u, 0u, 0u, 0u};
  };
  auto store_out = [&](int t, const float* src) {
#pragma unroll
    for (int q = 0; q < IOQ; ++q) {
      const int e = e0[q];
      if (el[q].real)
#pragma unroll
        for (int k = 0; k < S; ++k)
          st4(a.states, ((((long)k * B + el[q].b) * T + t) * N + tm.n) * D + el[q].d, p.dt_io,
              *reinterpret_cast<const f32x4*>(src + k * NE + e));
      if (training)
#pragma unroll
        for (int v = 0; v < NSAVE; ++v)
          *reinterpret_cast<f32x4*>(a.save + save_index(p, NE, t, tm.wgi, v, tm.team, e)) =
              *reinterpret_cast<const f32x4*>(src + (S + v) * NE + e);
    }
  };

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0);
  u32x4 buf[P][IOQ][GW];
#pragma unroll
  for (int j = 0; j < P; ++j)
    if (j < T) load_wx(j, buf[j]);
  for (int t0 = 0; t0 < T; t0 += P) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int t = t0 + j;
      if (t < T) {
#pragma unroll
        for (int q = 0; q < IOQ; ++q)
#pragma unroll
          for (int g = 0; g < GW; ++g)
            *reinterpret_cast<f32x4*>(xring + (j * GW + g) * NE + e0[q]) = raw4_f32(buf[j][q][g], p.dt_io);
        prof.mark(0);
        if (t + P < T) load_wx(t + P, buf[j]);
        prof.mark(1);
        __syncthreads();  // step t: Wx_t staged; outputs of step t-1 complete
        prof.mark(2);
        if (t >= 1) store_out(t - 1, ost + ((t - 1) & 1) * NOUT * NE);
        prof.mark(3);
      }
    }
  }
  __syncthreads();  // outputs of the last step complete
  store_out(T - 1, ost + ((T - 1) & 1) * NOUT * NE);
  prof.acc[5] = T;
  prof.flush(a.prof);
}

template <int CELL, int MMA, int KTW, int NB, int NDT, int KSC>
__global__ void __launch_bounds__(64 * (KSC + 1) * NDT) fwd_kernel(FwdArgs a) {
  using CS = CellShape<CELL>;
  constexpr int GR = CS::GR, GW = CS::GW, GT = CS::GT, S = CS::S;
  constexpr int NE = NB * 256, EPLMAX = 4 * NB / KSC, KS = KSC;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NOUT = S + NSAVE;
  const Plan& p = a.p;
  Team tm;
  if (!team_setup(p, tm, a.status)) return;
  const int D = p.D, B = p.B, T = p.T, N = p.N;

  extern __shared__ float lds[];
  float* red = lds + tm.team * Lds<CELL, NB>::fwd(KS);  // [2][KS][NB][GR][256]
  float* xring = red + 2L * KS * NB * GR * 256;         // [P][GW][NE]
  float* ost = xring + (long)kFwdRing * GW * NE;        // [2][NOUT][NE]

  // sLSTM: the reference's global predicate all(n0 == 0) over the call's whole initial state
  uint32_t zflag = 0;
  if constexpr (CELL == CELL_SLSTM) {
    int nz = 0;
    const long cnt = (long)B * N * D;
    for (long i = threadIdx.x; i < cnt; i += blockDim.x) nz |= ld_val(a.s0, 2 * cnt + i, p.dt_state) != 0.f;
    zflag = __syncthreads_or(nz) ? 0u : 1u;
  }
  if (tm.kw == KS) {
    fwd_io<CELL, MMA, NB>(a, tm, xring, ost);
    return;
  }

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
        const long base = (((long)g * N + tm.n) * D + tm.dt * 16 + tm.row) * D + (kt0 + j) * 32 + 8 * tm.kq;
#pragma unroll
        for (int i = 0; i < 8; ++i) frag_set(A[g][j], i, ld_val(a.R, base + i, p.dt_io));
      }
    }

  // ---- exchange word index of every run this wave reads (h_{t-1}[b][k])
  int xword[NB][KTW];
  bool bval[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int bl = bt * 16 + tm.row;
    bval[bt] = tm.slab * p.BS + bl < B;
#pragma unroll
    for (int j = 0; j < KTW; ++j) xword[bt][j] = (tm.group * p.BS + bl) * D + (kt0 + j) * 32 + 8 * tm.kq;
  }
  const int xpar = p.ngroups * p.BS * D;  // words per parity

  // ---- owned elements
  int oe[EPLMAX];
  bool own[EPLMAX];
  Elem el[EPLMAX];
  float st[EPLMAX][S], bias[EPLMAX][GT];
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    oe[s] = s * KS * 64 + tm.kw * 64 + tm.lane;
    own[s] = oe[s] < NE;
    el[s] = elem_of(p, tm, oe[s] & (NE - 1));
    el[s].real = el[s].real && own[s];
#pragma unroll
    for (int k = 0; k < S; ++k)
      st[s][k] = el[s].real ? ld_val(a.s0, (((long)k * B + el[s].b) * N + tm.n) * D + el[s].d, p.dt_state) : 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) bias[s][g] = own[s] ? ld_val(a.bias, ((long)g * N + tm.n) * D + el[s].d, p.dt_io) : 0.f;
  }

  Frag<MMA> X[NB][KTW];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt)
#pragma unroll
    for (int j = 0; j < KTW; ++j) X[bt][j].zero();

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0);

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
      const uint32_t polls = gather<MMA, NB, KTW>(xc, xword, bval, ((t - 1) & 1) * xpar, nkt, step_tag(t - 1), X,
                                                  a.status, a.spin_limit, abort);
      prof.add(4, polls);
    }
    prof.mark(0);

    // ---- 2. partial R . h over this wave's k-tiles, to LDS
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
    float* rp = red + (long)(t & 1) * KS * NB * GR * 256;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int g = 0; g < GR; ++g)
        *reinterpret_cast<f32x4*>(rp + (((tm.kw * NB + bt) * GR + g) * 64 + tm.lane) * 4) = acc[bt][g];
    prof.mark(1);
    __syncthreads();
    prof.mark(2);

    // ---- 3. owners: gates, cell, staged outputs, exchange
    const float* xr = xring + (long)(t % kFwdRing) * GW * NE;
    float* os = ost + (long)(t & 1) * NOUT * NE;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int e = oe[s];
      const int src = (e >> 8) * GR * 256 + mfma_pos(e);
      float ry[GR];
#pragma unroll
      for (int g = 0; g < GR; ++g) {
        float v = 0.f;
        #pragma unroll
        for (int w2 = 0; w2 < KS; ++w2) v += rp[w2 * NB * GR * 256 + src + g * 256];
        ry[g] = v;
      }
      float xcur[GW];
#pragma unroll
      for (int g = 0; g < GW; ++g) xcur[g] = xr[g * NE + e];
      float sv[NSAVE];
      if constexpr (CELL == CELL_GRU) {
        Cell<CELL_GRU>::fwd3(ry, xcur, bias[s], st[s], sv);
      } else {
        float g4[GR];
#pragma unroll
        for (int g = 0; g < GR; ++g) g4[g] = xcur[g] + ry[g] + bias[s][g];
        Cell<CELL>::fwd(g4, st[s], sv, (CELL == CELL_SLSTM && t == 0) ? zflag : 0u);
      }
      if (el[s].real && t + 1 < T)
        xstore<MMA>(xc, (t & 1) * xpar + ((long)tm.group * p.BS + el[s].bl) * D + el[s].d, st[s][0], step_tag(t));
#pragma unroll
      for (int k = 0; k < S; ++k) os[k * NE + e] = st[s][k];
#pragma unroll
      for (int v = 0; v < NSAVE; ++v) os[(S + v) * NE + e] = sv[v];
    }
    prof.mark(3);

  }
  __syncthreads();  // the I/O wave drains the last step

  // ---- carry: the last state in full precision
  if (a.carry) {
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
      if (el[s].real)
#pragma unroll
        for (int k = 0; k < S; ++k)
          st_val(a.carry, (((long)k * B + el[s].b) * N + tm.n) * D + el[s].d, p.dt_state, st[s][k]);
  }
  prof.acc[5] = T;
  prof.flush(a.prof);
}

// ===================================================================== backward
// I/O wave of a team: inputs (state cotangents, saved values) of iteration
// it+1 into the ring before barrier `it`; outputs of iteration `it` after it.
template <int CELL, int MMA, int NB>
__device__ void bwd_io(const BwdArgs& a, const Team& tm, float* iring, float* ost) {
  using CS = CellShape<CELL>;
  constexpr int GR = CS::GR, GW = CS::GW, S = CS::S, NE = NB * 256, IOQ = NB, P = BwdRing<CELL>::P;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NIN = S + NSAVE, NOUT = GW + (CELL == CELL_GRU ? 1 : 0);
  const Plan& p = a.p;
  const int T = p.T, N = p.N, D = p.D, B = p.B;
  const long wx_t = (long)GW * N * D;
  Elem el[IOQ];
  int e0[IOQ];
#pragma unroll
  for (int q = 0; q < IOQ; ++q) {
    e0[q] = io_elem(tm.lane, 4 * q);
    el[q] = elem_of(p, tm, e0[q]);
  }
  auto load_in = [&](int it, u32x4 (&dst)[IOQ][NIN]) {
    const int t = T - 1 - it;
#pragma unroll
    for (int q = 0; q < IOQ; ++q) {
#pragma unroll
      for (int k = 0; k < S; ++k)
        dst[q][k] = (el[q].real && a.d_states)
                        ? ld4_raw(a.d_states, ((((long)k * B + el[q].b) * T + t) * N + tm.n) * D + el[q].d, p.dt_io)
                        : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int v = 0; v < NSAVE; ++v)
        dst[q][S + v] = *reinterpret_cast<const u32x4*>(a.save + save_index(p, NE, t, tm.wgi, v, tm.team, e0[q]));
    }
  };
  auto stage = [&](int slot, const u32x4 (&src)[IOQ][NIN]) {
#pragma unroll
    for (int q = 0; q < IOQ; ++q) {
#pragma unroll
      for (int k = 0; k < S; ++k)
        *reinterpret_cast<f32x4*>(iring + ((long)slot * NIN + k) * NE + e0[q]) = raw4_f32(src[q][k], p.dt_io);
#pragma unroll
      for (int k = S; k < NIN; ++k) *reinterpret_cast<u32x4*>(iring + ((long)slot * NIN + k) * NE + e0[q]) = src[q][k];
    }
  };
  auto store_out = [&](int it, const float* src) {
    const int t = T - 1 - it;
#pragma unroll
    for (int q = 0; q < IOQ; ++q) {
      if (!el[q].real) continue;
#pragma unroll
      for (int g = 0; g < GW; ++g)
        st4(a.dwx, ((long)el[q].b * T + t) * wx_t + ((long)g * N + tm.n) * D + el[q].d, p.dt_io,
            *reinterpret_cast<const f32x4*>(src + g * NE + e0[q]));
      if constexpr (CELL == CELL_GRU)  // the R-only candidate gate's cotangent, for the dR GEMM
        *reinterpret_cast<f32x4*>(a.dcand + (((long)el[q].b * T + t) * N + tm.n) * D + el[q].d) =
            *reinterpret_cast<const f32x4*>(src + GW * NE + e0[q]);
    }
  };
  (void)NOUT;

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0);
  u32x4 buf[P][IOQ][NIN];
#pragma unroll
  for (int j = 0; j < P; ++j)
    if (j < T) load_in(j, buf[j]);
  stage(0, buf[0]);
  if (P < T) load_in(P, buf[0]);
  __syncthreads();  // iteration 0's inputs staged
  for (int it0 = 0; it0 < T; it0 += P) {
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int it = it0 + j;
      if (it < T) {
        const int jn = (j + 1) % P;
        if (it + 1 < T) {
          stage(jn, buf[jn]);
          prof.mark(0);
          if (it + 1 + P < T) load_in(it + 1 + P, buf[jn]);
          prof.mark(1);
        }
        __syncthreads();  // iteration it: outputs staged; inputs of it+1 staged
        prof.mark(2);
        store_out(it, ost + (long)(it & 1) * NOUT * NE);
        prof.mark(3);
      }
    }
  }
  prof.acc[5] = T;
  prof.flush(a.prof ? a.prof + 128 : nullptr);
}

template <int CELL, int MMA, int KTW, int NB, int NDT, int KSC>
__global__ void __launch_bounds__(64 * (KSC + 1) * NDT) bwd_kernel(BwdArgs a) {
  using CS = CellShape<CELL>;
  constexpr int GR = CS::GR, GW = CS::GW, GT = CS::GT, S = CS::S;
  constexpr int NE = NB * 256, EPLMAX = 4 * NB / KSC, KS = KSC;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NIN = S + NSAVE, P = BwdRing<CELL>::P;
  constexpr int NOUT = GW + (CELL == CELL_GRU ? 1 : 0);
  constexpr int NF = GR * KTW;  // max fragments of R^T per wave
  const Plan& p = a.p;
  Team tm;
  if (!team_setup(p, tm, a.status)) return;
  const int D = p.D, B = p.B, N = p.N, T = p.T;
  const int GD = GR * D;

  extern __shared__ float lds[];
  float* red = lds + tm.team * Lds<CELL, NB>::bwd(KS);  // [2][KS][NB][256]
  float* iring = red + 2L * KS * NB * 256;               // [P][NIN][NE]
  float* ost = iring + (long)P * NIN * NE;               // [2][NOUT][NE]

  if (tm.kw == KS) {
    bwd_io<CELL, MMA, NB>(a, tm, iring, ost);
    return;
  }

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
        frag_set(A[j], i, ld_val(a.R, (((long)g * N + tm.n) * D + o + i) * D + tm.dt * 16 + tm.row, p.dt_io));
    }
  }

  int xword[NB][NF];
  bool bval[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int bl = bt * 16 + tm.row;
    bval[bt] = tm.slab * p.BS + bl < B;
#pragma unroll
    for (int j = 0; j < NF; ++j) xword[bt][j] = (tm.group * p.BS + bl) * GD + (kt0 + j) * 32 + 8 * tm.kq;
  }
  const int xpar = p.ngroups * p.BS * GD;

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
      carry[s][k] = (el[s].real && a.d_carry)
                        ? ld_val(a.d_carry, (((long)k * B + el[s].b) * N + tm.n) * D + el[s].d, p.dt_state)
                        : 0.f;
    dhrec[s] = 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) dbacc[s][g] = 0.f;
  }

  Frag<MMA> X[NB][NF];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt)
#pragma unroll
    for (int j = 0; j < NF; ++j) X[bt][j].zero();

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0);
  __syncthreads();  // iteration 0's inputs staged by the I/O wave
  bool abort = false;
  for (int it = 0; it < T; ++it) {
    const int xoff = (it & 1) * xpar;
    // ---- 1. owners: pointwise backward of step t = T-1-it, publish dG_t
    const float* ir = iring + (long)(it % P) * NIN * NE;
    float* os = ost + (long)(it & 1) * NOUT * NE;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int e = oe[s];
      float ds[S];
#pragma unroll
      for (int k = 0; k < S; ++k) ds[k] = carry[s][k] + ir[k * NE + e];
      ds[0] += dhrec[s];
      float sv[NSAVE];
#pragma unroll
      for (int v = 0; v < NSAVE; ++v) sv[v] = ir[(S + v) * NE + e];
      float dry[GR], dwx[GW], db[GT], cr[S];
      Cell<CELL>::bwd(ds, sv, dry, dwx, db, cr);
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
#pragma unroll
        for (int g = 0; g < GR; ++g)
          xstore<MMA>(xc, xoff + ((long)tm.group * p.BS + el[s].bl) * GD + g * D + el[s].d, dry[g], step_tag(it));
      }
#pragma unroll
      for (int k = 0; k < S; ++k) carry[s][k] = cr[k];
#pragma unroll
      for (int g = 0; g < GW; ++g) os[g * NE + e] = dwx[g];
      if constexpr (CELL == CELL_GRU) os[GW * NE + e] = dry[0];
    }
    prof.mark(3);

    // ---- 2. dh_{t-1} partial = R^T dG_t over this wave's k-tiles
    const uint32_t polls = gather<MMA, NB, NF>(xc, xword, bval, xoff, nkt, step_tag(it), X, a.status,
                                               a.spin_limit, abort);
    prof.add(4, polls);
    prof.mark(0);
    f32x4 acc[NB];
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) acc[bt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NF; ++j)
      if (j < nkt) {
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) acc[bt] = mma(A[j], X[bt][j], acc[bt]);
      }
    float* rp = red + (long)(it & 1) * KS * NB * 256;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) *reinterpret_cast<f32x4*>(rp + ((tm.kw * NB + bt) * 64 + tm.lane) * 4) = acc[bt];
    prof.mark(1);
    __syncthreads();
    prof.mark(2);

    // ---- 3. owners: reduce -> recurrent cotangent of h_{t-1}
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int src = (oe[s] >> 8) * 256 + mfma_pos(oe[s]);
      float v = 0.f;
      #pragma unroll
      for (int w2 = 0; w2 < KS; ++w2) v += rp[w2 * NB * 256 + src];
      // the BF16 policy rounds the cotangent of the rounded hidden operand
      dhrec[s] = el[s].real ? (MMA == MMA_BF16 ? round_bf16(v) : v) : 0.f;
    }
    prof.mark(3);
  }

  // ---- d(initial state), d(bias) partials
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    if (!own[s]) continue;
    if (el[s].real) {
#pragma unroll
      for (int k = 0; k < S; ++k)
        st_val(a.ds0, (((long)k * B + el[s].b) * N + tm.n) * D + el[s].d, p.dt_state,
               carry[s][k] + (k == 0 ? dhrec[s] : 0.f));
    }
#pragma unroll
    for (int g = 0; g < GT; ++g)
      a.dbpart[(((long)tm.group * GT + g) * p.BS + el[s].bl) * D + el[s].d] = el[s].real ? dbacc[s][g] : 0.f;
  }
  prof.acc[5] = T;
  prof.flush(a.prof ? a.prof + 128 : nullptr);
}

}  // namespace frnn

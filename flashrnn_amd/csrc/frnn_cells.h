// Per-element cell arithmetic (FP32), forward and backward.
//
// Forward formulas follow flashrnn/flashrnn2/reference.py:84-113; the
// backward is the hand derivation of those formulas that the NumPy oracle
// (oracle/numpy_explicit.py) restates and checks against torch autograd,
// including torch's tie rule for maximum (half the cotangent to each side).
//
// Saved values per element and step (the "save" vector, FP32):
//   LSTM  : sig(i) sig(f) tanh(z) sig(o) tanh(c_t) c_{t-1}
//   GRU   : r u v cand h_{t-1}
//   Elman : h_t
//   sLSTM : sig(o) c_t n_t tanh(z) i' f' sig(-f) 8 w_m + 2 w_n
//           (w_n: share of the cotangent of max(npre, 1) that reaches npre;
//            w_m: share of the cotangent of m that reaches the input gate; each
//            is 0, 1/2 or 1, so the integer code holds both exactly). c_{t-1} and
//            n_{t-1} are not saved: they are c and n of step t-1 (the initial
//            state at t = 0), which the backward reads from that step's saves.
//
// Backward: prev holds (c_{t-1}, n_{t-1}) for the sLSTM; the other cells ignore it.
#pragma once

#include "frnn_device.h"

namespace frnn {

template <int CELL> struct Cell;

// ------------------------------------------------------------------- LSTM
template <> struct Cell<CELL_LSTM> {
  static constexpr int NSAVE = 6;
  // g: pre-activations (i, f, z, o) = Wx + Ry + b.  st: (h, c) in/out.
  __device__ __forceinline__ static void fwd(const float* g, float* st, float* sv, uint32_t) {
    const float si = sigmoidf_(g[0]), sf = sigmoidf_(g[1]), tz = tanhf_(g[2]), so = sigmoidf_(g[3]);
    const float c = sf * st[1] + si * tz;
    const float tc = tanhf_(c);
    sv[0] = si; sv[1] = sf; sv[2] = tz; sv[3] = so; sv[4] = tc; sv[5] = st[1];
    st[0] = so * tc;
    st[1] = c;
  }
  // ds: total cotangents of (h_t, c_t). Out: dry (= dWx), cotangent carried to
  // (h_{t-1}, c_{t-1}) through direct (non-recurrent) paths.
  __device__ __forceinline__ static void bwd(const float* ds, const float* sv, const float*, float* dry, float* dwx,
                                             float* db, float* carry, bool v1) {
    const float si = sv[0], sf = sv[1], tz = sv[2], so = sv[3], tc = sv[4], cp = sv[5];
    const float dh = ds[0];
    const float dc = ds[1] + dh * so * (1.f - tc * tc);
    dry[0] = dc * tz * si * (1.f - si);
    dry[1] = dc * cp * sf * (1.f - sf);
    dry[2] = dc * si * (1.f - tz * tz);
    dry[3] = dh * tc * so * (1.f - so);
#pragma unroll
    for (int k = 0; k < 4; ++k) { dwx[k] = dry[k]; db[k] = dry[k]; }
    carry[0] = 0.f;
    carry[1] = dc * sf;
  }
};

// -------------------------------------------------------------------- GRU
// Input gates (r, u, v), recurrent gates (cand, r, u), biases (cand, r, u, v).
template <> struct Cell<CELL_GRU> {
  static constexpr int NSAVE = 5;
  // g layout: g[0..2] = Ry(cand, r, u); x[0..2] = Wx(r, u, v); b[0..3].
  __device__ __forceinline__ static void fwd3(const float* ry, const float* x, const float* b, float* st,
                                              float* sv) {
    const float cand = ry[0] + b[0];
    const float r = sigmoidf_(x[0] + ry[1] + b[1]);
    const float u = sigmoidf_(x[1] + ry[2] + b[2]);
    const float v = tanhf_(x[2] + b[3] + r * cand);
    sv[0] = r; sv[1] = u; sv[2] = v; sv[3] = cand; sv[4] = st[0];
    st[0] = u * st[0] + (1.f - u) * v;
  }
  __device__ __forceinline__ static void bwd(const float* ds, const float* sv, const float*, float* dry, float* dwx,
                                             float* db, float* carry, bool v1) {
    const float r = sv[0], u = sv[1], v = sv[2], cand = sv[3], hp = sv[4];
    const float dh = ds[0];
    const float dva = dh * (1.f - u) * (1.f - v * v);
    const float dcand = dva * r;
    const float dra = dva * cand * r * (1.f - r);
    const float dua = dh * (hp - v) * u * (1.f - u);
    dry[0] = dcand; dry[1] = dra; dry[2] = dua;
    dwx[0] = dra; dwx[1] = dua; dwx[2] = dva;
    db[0] = dcand; db[1] = dra; db[2] = dua; db[3] = dva;
    carry[0] = dh * u;
  }
};

// ------------------------------------------------------------------ Elman
template <> struct Cell<CELL_ELMAN> {
  static constexpr int NSAVE = 1;
  __device__ __forceinline__ static void fwd(const float* g, float* st, float* sv, uint32_t) {
    st[0] = tanhf_(g[0]);
    sv[0] = st[0];
  }
  __device__ __forceinline__ static void bwd(const float* ds, const float* sv, const float*, float* dry, float* dwx,
                                             float* db, float* carry, bool v1) {
    const float h = sv[0];
    const float da = ds[0] * (1.f - h * h);
    dry[0] = da; dwx[0] = da; db[0] = da;
    carry[0] = 0.f;
  }
};

// ------------------------------------------------------------------ sLSTM
template <> struct Cell<CELL_SLSTM> {
  static constexpr int NSAVE = 8;
  // st: (h, c, n, m). zero: the global all-normalizers-zero predicate of this step.
  __device__ __forceinline__ static void fwd(const float* g, float* st, float* sv, uint32_t zero) {
    const float gi = g[0], gf = g[1], gz = g[2], go = g[3];
    const float lf = logsigmoidf_(gf) + st[3];
    float m, wm;
    if (zero) { m = gi; wm = 1.f; }
    else {
      m = fmaxf(gi, lf);
      wm = gi > lf ? 1.f : (gi == lf ? 0.5f : 0.f);
    }
    const float ia = fexp(gi - m), fa = fexp(lf - m);
    const float tz = tanhf_(gz), so = sigmoidf_(go);
    const float c = fa * st[1] + ia * tz;
    const float npre = fa * st[2] + ia;
    const float nn = fmaxf(npre, 1.f);
    const float wn = npre > 1.f ? 1.f : (npre == 1.f ? 0.5f : 0.f);
    sv[0] = so; sv[1] = c; sv[2] = nn; sv[3] = tz; sv[4] = ia; sv[5] = fa;
    sv[6] = sigmoidf_(-gf); sv[7] = 8.f * wm + 2.f * wn;
    st[0] = so * c / nn;
    st[1] = c;
    st[2] = nn;
    st[3] = m;
  }
  __device__ __forceinline__ static void bwd(const float* ds, const float* sv, const float* prev, float* dry,
                                             float* dwx, float* db, float* carry, bool v1) {
    const float so = sv[0], c = sv[1], nn = sv[2], tz = sv[3], ia = sv[4], fa = sv[5];
    const float cold = prev[0], nold = prev[1], sgn = sv[6];
    const float wq = floorf(0.25f * sv[7]);  // 2 w_m (sv[7] = 4 (2 w_m) + 2 w_n, an integer)
    const float wm = 0.5f * wq, wn = 0.5f * (sv[7] - 4.f * wq);
    const float dh = ds[0];
    const float rn = 1.f / nn;
    const float dgo = dh * c * rn * so * (1.f - so);
    const float dc = ds[1] + dh * so * rn;
    const float dn = ds[2] - dh * so * c * rn * rn;
    // v1 (FlashRNN v1 / FlashRNN2 training convention): the normalizer clamp passes
    // its cotangent straight through and the stabilizer m carries none
    const float dnpre = v1 ? dn : dn * wn;
    const float dfa = dc * cold + dnpre * nold;
    const float dia = dc * tz + dnpre;
    const float dgz = dc * ia * (1.f - tz * tz);
    float dgi = dia * ia;
    float dlf = dfa * fa;
    if (!v1) {
      const float dm = ds[3] - dia * ia - dfa * fa;
      dgi += dm * wm;
      dlf += dm * (1.f - wm);
    }
    const float dgf = dlf * sgn;
    dry[0] = dgi; dry[1] = dgf; dry[2] = dgz; dry[3] = dgo;
#pragma unroll
    for (int k = 0; k < 4; ++k) { dwx[k] = dry[k]; db[k] = dry[k]; }
    carry[0] = 0.f;
    carry[1] = dc * fa;
    carry[2] = dnpre * fa;
    carry[3] = v1 ? 0.f : dlf;
  }
};

}  // namespace frnn

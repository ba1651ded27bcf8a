// dR GEMM, its split-K / bias reduction, and the exchange clear.
//
// Reference counterparts (behaviour, not code):
//   dR GEMM        flashrnn/flashrnn/fused/flashrnn_fused_backward.cu:1050-1056 (cuBLAS there)
//   db reduction   flashrnn/flashrnn/fused/flashrnn_fused_backward.cu:627-666
#include "frnn_device.h"
#include "frnn_kernels.h"
#include "frnn_plan.h"

namespace frnn {

// ============================================================== dR GEMM
// part[split][n][m][q] = sum over this split's k of dG[n][k][m] * h[n][k][q],
// m = (g, o) in [0, GR*D), q in [0, D), k = (t, b) in chunks of 8 batch rows.
// One wave computes a 32x32 tile; operands are read as 16-byte runs straight
// from the chunked layouts (8 consecutive k per lane), no LDS needed.
template <int MMA>
__device__ __forceinline__ void gemm_frag(const void* base, long run, bool valid, Frag<MMA>& f) {
  if constexpr (MMA == MMA_BF16) {
    u16x8 v = valid ? static_cast<const u16x8*>(base)[run] : u16x8{};
    f.v = __builtin_bit_cast(bf16x8, v);
  } else {
    const f32x4* q = static_cast<const f32x4*>(base) + 2 * run;
    f32x4 lo = valid ? q[0] : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 hi = valid ? q[1] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) { f.v[i] = lo[i]; f.v[4 + i] = hi[i]; }
  }
}

template <int MMA>
__global__ void __launch_bounds__(256) dr_gemm_kernel(GemmArgs a) {
  const Plan& p = a.p;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int GD = p.GR * p.D;
  const int mt = GD / 32, qt = p.D / 32;
  const int tiles = p.N * mt * qt;
  if (wave >= tiles * p.splitk) return;
  const int split = wave / tiles;
  int rem = wave % tiles;
  const int n = rem / (mt * qt);
  rem %= mt * qt;
  const int m0 = (rem / qt) * 32, q0 = (rem % qt) * 32;
  const long KC = (long)p.T * (p.Bp8 / 8);  // chunks of 8 along k
  const long KTT = (KC + 3) / 4;            // 32-wide k-tiles
  const long kt_lo = KTT * split / p.splitk, kt_hi = KTT * (split + 1) / p.splitk;
  const int row = lane & 15, kq = lane >> 4;
  const long dg0 = (long)n * KC * GD, hs0 = (long)n * KC * p.D;  // in 8-element runs
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (long kt = kt_lo; kt < kt_hi; ++kt) {
    const long c = kt * 4 + kq;
    Frag<MMA> fa[2], fb[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      gemm_frag<MMA>(a.dgsave, dg0 + c * GD + m0 + i * 16 + row, c < KC, fa[i]);
      gemm_frag<MMA>(a.hsave, hs0 + c * p.D + q0 + i * 16 + row, c < KC, fb[i]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mma(fa[i], fb[j], acc[i][j]);
  }
  float* out = a.part + ((long)split * p.N + n) * GD * p.D;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[(long)(m0 + i * 16 + 4 * kq + r) * p.D + q0 + j * 16 + row] = acc[i][j][r];
}

// dR = sum of the split-K partials (layout [n][g*D+o][p] -> [g][n][o][p]);
// db = sum of the per-group partials over slabs and batch rows.
__global__ void __launch_bounds__(256) dr_reduce_kernel(GemmArgs a) {
  const Plan& p = a.p;
  const long GD = (long)p.GR * p.D;
  const long ndr = (long)p.N * GD * p.D;
  const long ndb = (long)p.GT * p.N * p.D;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < ndr + ndb; i += (long)gridDim.x * 256) {
    if (i < ndr) {
      const long q = i % p.D, m = (i / p.D) % GD, n = i / (p.D * GD);
      float v = 0.f;
      for (int s = 0; s < p.splitk; ++s) v += a.part[(((long)s * p.N + n) * GD + m) * p.D + q];
      const long g = m / p.D, o = m % p.D;
      st_val(a.dR, ((g * p.N + n) * p.D + o) * p.D + q, p.dt_io, v);
    } else {
      const long j = i - ndr;
      const long d = j % p.D, n = (j / p.D) % p.N, g = j / ((long)p.D * p.N);
      float v = 0.f;
      for (int sl = 0; sl < p.nslab; ++sl)
        for (int bl = 0; bl < p.BS; ++bl) v += a.dbpart[(((n * p.nslab + sl) * p.GT + g) * p.BS + bl) * p.D + d];
      st_val(a.db, (g * p.N + n) * p.D + d, p.dt_io, v);
    }
  }
}

__global__ void __launch_bounds__(256) clear_kernel(uint32_t* p, long n) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) p[i] = 0u;
}

const void* gemm_kernel(int mma) {
  return mma == MMA_BF16 ? reinterpret_cast<const void*>(&dr_gemm_kernel<MMA_BF16>)
                         : reinterpret_cast<const void*>(&dr_gemm_kernel<MMA_F32>);
}
const void* reduce_kernel() { return reinterpret_cast<const void*>(&dr_reduce_kernel); }
const void* zero_kernel() { return reinterpret_cast<const void*>(&clear_kernel); }

}  // namespace frnn

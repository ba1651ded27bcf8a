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
// One workgroup (one wave) computes a 32x32 tile of part[split][n][m][q] over
// its share of k = (b, t): m = g*D + o indexes the recurrent gate
// cotangents, q the previous hidden state. Operands are read where the
// recurrence left them -- dG from dWx (GRU gate 0: the candidate buffer),
// h_{t-1} from the state output (h_{-1} from s0) -- in runs of 8 contiguous
// m or q, and transposed through LDS so each MFMA fragment is one 16-byte
// (bf16) or two 16-byte (f32) LDS reads with 8 consecutive k.
template <int MMA> struct GemmElem { typedef unsigned short type; };
template <> struct GemmElem<MMA_F32> { typedef float type; };

template <int MMA>
__device__ __forceinline__ typename GemmElem<MMA>::type gemm_cvt(float v) {
  if constexpr (MMA == MMA_BF16) return (unsigned short)bf16_bits(v);
  else return v;
}

template <int MMA>
__device__ __forceinline__ void gemm_frag(const typename GemmElem<MMA>::type* row, Frag<MMA>& f) {
  if constexpr (MMA == MMA_BF16) {
    f.v = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(row));
  } else {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(row);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(row + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { f.v[i] = lo[i]; f.v[4 + i] = hi[i]; }
  }
}

template <int MMA>
__global__ void __launch_bounds__(64) dr_gemm_kernel(GemmArgs a) {
  typedef typename GemmElem<MMA>::type E;
  constexpr int LD = 40;  // LDS row stride (32 k + pad), elements
  __shared__ __attribute__((aligned(16))) E As[32 * LD];
  __shared__ __attribute__((aligned(16))) E Hs[32 * LD];
  const Plan& p = a.p;
  const int lane = threadIdx.x;
  const int GD = p.GR * p.D;
  const int mt = GD / 32, qt = p.D / 32;
  const int tiles = p.N * mt * qt;
  const int split = blockIdx.x / tiles;
  int rem = blockIdx.x % tiles;
  const int n = rem / (mt * qt);
  rem %= mt * qt;
  const int m0 = (rem / qt) * 32, q0 = (rem % qt) * 32;
  const int B = p.B, T = p.T, N = p.N, D = p.D;
  const long K = (long)B * T;
  const long KT = (K + 31) / 32;
  const long k_lo = 32 * (KT * split / p.splitk), k_hi = 32 * (KT * (split + 1) / p.splitk);
  const long wx_t = (long)p.GW * N * D;
  const int row = lane & 15, kq = lane >> 4;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (long k0 = k_lo; k0 < k_hi; k0 += 32) {
    // 32 k x 32 columns per operand = 128 runs of 8; two per lane and operand
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int c = lane + 64 * r;
      const int kl = c >> 2, col = (c & 3) * 8;
      const long k = k0 + kl;
      f32x4 va0 = {0.f, 0.f, 0.f, 0.f}, va1 = va0, vh0 = va0, vh1 = va0;
      if (k < K) {
        const long b = k / T, t = k % T;
        const int m = m0 + col, g = m / D, o = m % D;
        if (p.cell == CELL_GRU && g == 0) {
          const float* src = a.dcand + ((b * T + t) * N + n) * D + o;
          va0 = *reinterpret_cast<const f32x4*>(src);
          va1 = *reinterpret_cast<const f32x4*>(src + 4);
        } else {
          const int gw = p.cell == CELL_GRU ? g - 1 : g;
          const long i = (b * T + t) * wx_t + ((long)gw * N + n) * D + o;
          va0 = ld4(a.dwx, i, p.dt_io);
          va1 = ld4(a.dwx, i + 4, p.dt_io);
        }
        const int q = q0 + col;
        if (t == 0) {
          const long i = (b * N + n) * D + q;  // h_{-1} = s0[0]
          vh0 = ld4(a.s0, i, p.dt_state);
          vh1 = ld4(a.s0, i + 4, p.dt_state);
        } else {
          const long i = ((b * T + t - 1) * N + n) * D + q;  // h_{t-1} = states[0][b][t-1]
          vh0 = ld4(a.states, i, p.dt_io);
          vh1 = ld4(a.states, i + 4, p.dt_io);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        As[(col + i) * LD + kl] = gemm_cvt<MMA>(va0[i]);
        As[(col + 4 + i) * LD + kl] = gemm_cvt<MMA>(va1[i]);
        Hs[(col + i) * LD + kl] = gemm_cvt<MMA>(vh0[i]);
        Hs[(col + 4 + i) * LD + kl] = gemm_cvt<MMA>(vh1[i]);
      }
    }
    __syncthreads();
    Frag<MMA> fa[2], fh[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      gemm_frag<MMA>(As + (i * 16 + row) * LD + 8 * kq, fa[i]);
      gemm_frag<MMA>(Hs + (i * 16 + row) * LD + 8 * kq, fh[i]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mma(fa[i], fh[j], acc[i][j]);
    __syncthreads();
  }
  float* out = a.part + ((long)split * N + n) * GD * D;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) out[(long)(m0 + i * 16 + 4 * kq + r) * D + q0 + j * 16 + row] = acc[i][j][r];
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

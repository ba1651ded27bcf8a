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
  if constexpr (MMA != MMA_F32) return (unsigned short)op_bits<MMA>(v);
  else return v;
}

template <int MMA>
__device__ __forceinline__ void gemm_frag(const typename GemmElem<MMA>::type* row, Frag<MMA>& f) {
  if constexpr (MMA == MMA_BF16) {
    f.v = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8*>(row));
  } else if constexpr (MMA == MMA_F16) {
    f.v = __builtin_bit_cast(f16x8, *reinterpret_cast<const u16x8*>(row));
  } else {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(row);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(row + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { f.v[i] = lo[i]; f.v[4 + i] = hi[i]; }
  }
}

// Operand runs of 8 contiguous columns for k = (b, t): dG (m = g*D + o) and
// h_{t-1} (q). A run's column offset is fixed for the whole kernel and its k
// advances by a constant per stage, so the (b, t) of a run is carried from
// stage to stage instead of being divided out of k each time.
struct GemmRunA {  // dG run: columns m .. m+7 of k = (b, t)
  const void* base;  // dwx (or the GRU candidate buffer) at this run's column, k = 0
  bool f32;          // the candidate buffer (FP32), else dwx in dt_io
  long kstride;      // elements between consecutive t
  int b, t;
};
struct GemmRunH {  // h_{t-1} run: columns q .. q+7
  int b, t;
};

__device__ __forceinline__ void gemm_advance(int& b, int& t, int dk, int T) {
  t += dk;
  while (t >= T) {
    t -= T;
    ++b;
  }
}

// Workgroup tile (32*WM) x (32*WQ) of part[split][n][m][q], WM*WQ waves of 32x32
// each; k in steps of 32 through double-buffered LDS, the next step's global
// loads in flight while the current step runs on MFMA. Operands are written to
// LDS transposed ([column][k]) so each MFMA fragment is one 16-byte (bf16) or
// two 16-byte (f32) reads of 8 consecutive k.
// KSUB: 32-wide k sub-steps per stage (2 and 3 measured no faster than 1 at
// the LSTM B8 T1024 N3 D256 shape).
template <int MMA, int WM, int WQ, int KSUB>
__global__ void __launch_bounds__(64 * WM * WQ) dr_gemm_kernel(GemmArgs a) {
  typedef typename GemmElem<MMA>::type E;
  constexpr int KW = 32 * KSUB;          // k per stage
  constexpr int LD = KW + 8;             // LDS row stride (KW k + pad), elements
  constexpr int NT = 64 * WM * WQ;       // threads
  constexpr int RA = KW * WM * 4 / NT;   // runs of 8 per thread per stage: A (KW k x 32*WM m / 8)
  constexpr int RH = KW * WQ * 4 / NT;   // and h
  __shared__ __attribute__((aligned(16))) E As[2][32 * WM * LD];
  __shared__ __attribute__((aligned(16))) E Hs[2][32 * WQ * LD];
  const Plan& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int GD = p.GR * p.D;
  const int mt = GD / (32 * WM), qt = p.D / (32 * WQ);
  const int tiles = p.N * mt * qt;
  // XCD-major tile order: workgroup b runs on XCD b % 8, so consecutive tiles
  // (the m-tiles of one h block, then the q-tiles of one dG block) go to one
  // XCD and share its L2 instead of being fetched once per XCD.
  const int full = (int)(gridDim.x / kXcds) * kXcds, bx = blockIdx.x;
  const int tile_id = bx < full ? (bx % kXcds) * (full / kXcds) + bx / kXcds : bx;
  const int split = tile_id / tiles;
  int rem = tile_id % tiles;
  const int n = rem / (mt * qt);
  rem %= mt * qt;
  const int m0 = (rem % mt) * 32 * WM, q0 = (rem / mt) * 32 * WQ;  // m-tiles of one q block adjacent
  const long K = (long)p.B * p.T;
  const long KT = (K + KW - 1) / KW;
  const long s_lo = KT * split / p.splitk, s_hi = KT * (split + 1) / p.splitk;
  const int row = lane & 15, kq = lane >> 4;
  const int wm = w % WM, wq = w / WM;

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // per-thread runs: A run c -> (k = c / (4*WM), column 8*(c % (4*WM))), h likewise with WQ
  const long K0 = (long)KW * s_lo;
  const long wxt = (long)p.GW * p.N * p.D;  // dwx elements per (b, t)
  GemmRunA ga[RA];
  GemmRunH gh[RH];
#pragma unroll
  for (int r = 0; r < RA; ++r) {
    const int c = tid + NT * r, m = m0 + 8 * (c % (4 * WM));
    const long k = K0 + c / (4 * WM);
    ga[r].b = (int)(k / p.T);
    ga[r].t = (int)(k % p.T);
    const int g = m / p.D, o = m % p.D;
    if (p.cell == CELL_GRU && g == 0) {
      ga[r].base = a.dcand + (long)n * p.D + o;
      ga[r].f32 = true;
      ga[r].kstride = (long)p.N * p.D;
    } else {
      const int gw = p.cell == CELL_GRU ? g - 1 : g;
      ga[r].base = static_cast<const char*>(a.dwx) + (((long)gw * p.N + n) * p.D + o) * (p.dt_io == DT_F32 ? 4 : 2);
      ga[r].f32 = false;
      ga[r].kstride = wxt;
    }
  }
#pragma unroll
  for (int r = 0; r < RH; ++r) {
    const int c = tid + NT * r;
    const long k = K0 + c / (4 * WQ);
    gh[r].b = (int)(k / p.T);
    gh[r].t = (int)(k % p.T);
  }
  f32x4 ra[RA][2], rh[RH][2];
  auto fetch = [&]() {  // the runs' current (b, t); then advance them one stage
#pragma unroll
    for (int r = 0; r < RA; ++r) {
      const int c = tid + NT * r, b = ga[r].b, t = ga[r].t;
      ra[r][0] = ra[r][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (b < p.B) {
        const long i = ((long)b * p.T + t) * ga[r].kstride;
        if (ga[r].f32) {
          const float* src = static_cast<const float*>(ga[r].base) + i;
          ra[r][0] = *reinterpret_cast<const f32x4*>(src);
          ra[r][1] = *reinterpret_cast<const f32x4*>(src + 4);
        } else {
          ra[r][0] = ld4(ga[r].base, i, p.dt_io);
          ra[r][1] = ld4(ga[r].base, i + 4, p.dt_io);
        }
      }
      gemm_advance(ga[r].b, ga[r].t, KW, p.T);
      (void)c;
    }
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const int c = tid + NT * r, q = q0 + 8 * (c % (4 * WQ)), b = gh[r].b, t = gh[r].t;
      rh[r][0] = rh[r][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (b < p.B) {
        if (t == 0) {
          const long i = ((long)b * p.N + n) * p.D + q;  // h_{-1} = s0[0]
          rh[r][0] = ld4(a.s0, i, p.dt_state);
          rh[r][1] = ld4(a.s0, i + 4, p.dt_state);
        } else {
          const long i = (((long)b * p.T + t - 1) * p.N + n) * p.D + q;  // h_{t-1} = states[0][b][t-1]
          rh[r][0] = ld4(a.states, i, p.dt_out);
          rh[r][1] = ld4(a.states, i + 4, p.dt_out);
        }
      }
      gemm_advance(gh[r].b, gh[r].t, KW, p.T);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int r = 0; r < RA; ++r) {
      const int c = tid + NT * r, kl = c / (4 * WM), col = 8 * (c % (4 * WM));
#pragma unroll
      for (int i = 0; i < 8; ++i) As[buf][(col + i) * LD + kl] = gemm_cvt<MMA>(ra[r][i / 4][i % 4]);
    }
#pragma unroll
    for (int r = 0; r < RH; ++r) {
      const int c = tid + NT * r, kl = c / (4 * WQ), col = 8 * (c % (4 * WQ));
#pragma unroll
      for (int i = 0; i < 8; ++i) Hs[buf][(col + i) * LD + kl] = gemm_cvt<MMA>(rh[r][i / 4][i % 4]);
    }
  };

  if (s_lo < s_hi) {
    fetch();
    stage(0);
    __syncthreads();
  }
  for (long s = s_lo; s < s_hi; ++s) {
    const int buf = (int)((s - s_lo) & 1);
    if (s + 1 < s_hi) fetch();
#pragma unroll
    for (int ks = 0; ks < KSUB; ++ks) {
      Frag<MMA> fa[2], fh[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        gemm_frag<MMA>(As[buf] + (wm * 32 + i * 16 + row) * LD + 32 * ks + 8 * kq, fa[i]);
        gemm_frag<MMA>(Hs[buf] + (wq * 32 + i * 16 + row) * LD + 32 * ks + 8 * kq, fh[i]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mma(fa[i], fh[j], acc[i][j]);
    }
    if (s + 1 < s_hi) stage(buf ^ 1);
    __syncthreads();
  }
  float* out = a.part + ((long)split * p.N + n) * GD * p.D;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[(long)(m0 + wm * 32 + i * 16 + 4 * kq + r) * p.D + q0 + wq * 32 + j * 16 + row] = acc[i][j][r];
}

// The same 64x64 tiles and split-K stages of 32 k, with the operand tiles
// loaded by LDS-DMA (global_load_lds: no registers in flight) into a ring of
// kGemmRing stages, kGemmRing - 1 stages ahead of their use: the register-
// staged kernel above waits a full load latency per stage. Wave w loads rows
// 8w .. 8w+7 of a stage (k = 32 s + 8w + lane / 8, 16 bytes = 8 columns per
// lane) of both operands, straight from dWx and from the state output (s0 for
// t = 0) in their [k][column] layout; a rows beyond B*T reads 16 zero bytes.
// A fragment then gathers its 8 consecutive k of one column with 16-bit LDS
// reads (one per k), which a row-major tile needs. Same stages, same k
// grouping per MFMA, so the result is bitwise that of the kernel above.
constexpr int kGemmRing = 4;
constexpr int kGemmGroup = 8 * 128 + 64;                 // bytes per 8-row group (+ pad against bank conflicts)
constexpr int kGemmSlot = 2 * 4 * kGemmGroup;            // A and h, four groups each

template <int MMA>
__device__ __forceinline__ Frag<MMA> gemm_gather(const char* grp, int col) {
  // 8 k (rows j of the 8-row group) of column col, packed two per dword
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 v;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const uint32_t lo = *reinterpret_cast<const unsigned short*>(grp + j * 128 + 2 * col);
    const uint32_t hi = *reinterpret_cast<const unsigned short*>(grp + (j + 1) * 128 + 2 * col);
    v[j / 2] = (int)(lo | (hi << 16));
  }
  Frag<MMA> f;
  if constexpr (MMA == MMA_BF16) f.v = __builtin_bit_cast(bf16x8, v);
  else f.v = __builtin_bit_cast(f16x8, v);
  return f;
}

template <int MMA>
__global__ void __launch_bounds__(256) dr_gemm_dma_kernel(GemmArgs a) {
  static_assert(MMA != MMA_F32, "16-bit operands only");
  __shared__ __attribute__((aligned(16))) char ring[kGemmRing * kGemmSlot];
  const Plan& p = a.p;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int GD = p.GR * p.D;
  const int mt = GD / 64, qt = p.D / 64;
  const int tiles = p.N * mt * qt;
  const int full = (int)(gridDim.x / kXcds) * kXcds, bx = blockIdx.x;
  const int tile_id = bx < full ? (bx % kXcds) * (full / kXcds) + bx / kXcds : bx;
  const int split = tile_id / tiles;
  int rem = tile_id % tiles;
  const int n = rem / (mt * qt);
  rem %= mt * qt;
  const int m0 = (rem % mt) * 64, q0 = (rem / mt) * 64;
  const long K = (long)p.B * p.T;
  const long KT = (K + 31) / 32;
  const long s_lo = KT * split / p.splitk, s_hi = KT * (split + 1) / p.splitk;
  const int row = lane & 15, kq = lane >> 4;
  const int wm = w & 1, wq = w >> 1;

  // this lane's DMA row: k = 32 s + 8 w + lane / 8, columns 8 (lane % 8) .. +7
  const int g = m0 / p.D, o = m0 % p.D + 8 * (lane & 7), q = q0 + 8 * (lane & 7);
  // A rows: dWx at gate g (GRU: gate g - 1 of dWx, gate 0 the candidate cotangents)
  const bool cand = p.cell == CELL_GRU && g == 0;
  const long wxt = cand ? (long)p.N * p.D : (long)p.GW * p.N * p.D;  // elements per (b, t)
  const char* abase = cand ? static_cast<const char*>(a.dcand16) + ((long)n * p.D + o) * 2
                           : static_cast<const char*>(a.dwx) +
                                 (((long)(p.cell == CELL_GRU ? g - 1 : g) * p.N + n) * p.D + o) * 2;
  const char* sbase = static_cast<const char*>(a.states) + ((long)n * p.D + q) * 2;  // + ((b T + t - 1) N D) * 2
  const char* s0base = static_cast<const char*>(a.s0) + ((long)n * p.D + q) * 2;     // + (b N D) * 2
  long k = 32 * s_lo + 8 * w + (lane >> 3);
  int b = (int)(k / p.T), t = (int)(k % p.T);
  auto issue = [&](long s) {  // DMA of stage s into its ring slot; advances this lane's row
    char* slot = ring + (int)(s % kGemmRing) * kGemmSlot;
    const char* src_a = static_cast<const char*>(a.zero);
    const char* src_h = static_cast<const char*>(a.zero);
    if (b < p.B) {
      src_a = abase + ((long)b * p.T + t) * wxt * 2;
      src_h = t > 0 ? sbase + ((long)b * p.T + t - 1) * p.N * p.D * 2 : s0base + (long)b * p.N * p.D * 2;
    }
    __builtin_amdgcn_global_load_lds(src_a, (__attribute__((address_space(3))) void*)(slot + w * kGemmGroup), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(src_h, (__attribute__((address_space(3))) void*)(slot + (4 + w) * kGemmGroup), 16,
                                     0, 0);
    t += 32;
    while (t >= p.T) {
      t -= p.T;
      ++b;
    }
  };

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int AHEAD = kGemmRing - 1;
  for (long s = s_lo; s < s_lo + AHEAD && s < s_hi; ++s) issue(s);
  for (long s = s_lo; s < s_hi; ++s) {
    // this wave's loads of stage s have landed: 2 DMAs per later stage may still fly
    if (s + AHEAD <= s_hi) wait_vm<2 * (AHEAD - 1)>();
    else wait_vm<0>();
    // every wave's loads of stage s landed; everyone done with stage s-1 (a
    // plain barrier: a fence here would also wait for the later stages' DMA)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (s + AHEAD < s_hi) issue(s + AHEAD);  // into the slot of stage s-1
    const char* slot = ring + (int)(s % kGemmRing) * kGemmSlot;
    Frag<MMA> fa[2], fh[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      fa[i] = gemm_gather<MMA>(slot + kq * kGemmGroup, wm * 32 + i * 16 + row);
      fh[i] = gemm_gather<MMA>(slot + (4 + kq) * kGemmGroup, wq * 32 + i * 16 + row);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mma(fa[i], fh[j], acc[i][j]);
  }
  float* out = a.part + ((long)split * p.N + n) * GD * p.D;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        out[(long)(m0 + wm * 32 + i * 16 + 4 * kq + r) * p.D + q0 + wq * 32 + j * 16 + row] = acc[i][j][r];
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

// FP32 -> 16-bit (dt: BF16 or FP16) bits, round to nearest even.
__global__ void __launch_bounds__(256) to16_copy_kernel(const float* src, unsigned short* dst, long n, int dt) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256)
    dst[i] = (unsigned short)h16_bits(src[i], dt);
}

__global__ void __launch_bounds__(256) clear_kernel(uint32_t* p, long n) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) p[i] = 0u;
}

template <int MMA>
static const void* gemm_of(bool wide) {
  return wide ? reinterpret_cast<const void*>(&dr_gemm_kernel<MMA, 2, 2, 1>)
              : reinterpret_cast<const void*>(&dr_gemm_kernel<MMA, 1, 1, 1>);
}
const void* gemm_kernel(int mma, bool wide) {
  switch (mma) {
    case MMA_BF16: return gemm_of<MMA_BF16>(wide);
    case MMA_F16: return gemm_of<MMA_F16>(wide);
    case MMA_F32: return gemm_of<MMA_F32>(wide);
  }
  return nullptr;
}
const void* gemm_dma_kernel(int mma) {
  switch (mma) {
    case MMA_BF16: return reinterpret_cast<const void*>(&dr_gemm_dma_kernel<MMA_BF16>);
    case MMA_F16: return reinterpret_cast<const void*>(&dr_gemm_dma_kernel<MMA_F16>);
  }
  return nullptr;
}
const void* reduce_kernel() { return reinterpret_cast<const void*>(&dr_reduce_kernel); }
const void* zero_kernel() { return reinterpret_cast<const void*>(&clear_kernel); }
const void* to16_kernel() { return reinterpret_cast<const void*>(&to16_copy_kernel); }

}  // namespace frnn

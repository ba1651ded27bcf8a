// Input projection Wx = x W^T, computed by workgroups that run beside the
// forward recurrence in the same launch (or alone, before it).
//
// The reference leaves this GEMM to its caller ("Typically the inputs are
// modified with a linear layer which is omitted here", README.md:17); its
// layer (flashrnn/flashrnn2/torch_layer.py:14-80) runs it as a separate
// library call before the recurrence. Here the recurrence occupies
// N * ceil(B/16) * D/16 CUs and the projection runs on the others: the
// recurrence's I/O waves wait, per step, for the rows of Wx that step reads.
//
//   x   [B][T][I]            (16-bit, the MMA's type)
//   W   [G_W*N*D][I]          the reference layer's [G,N,D,I] weight, flattened
//   Wx  [B][T][G_W*N*D]       the recurrence's input layout [B,T,G_W,N,D]
//
// Output rows are ordered by time: row m = t*B + b. A tile is 64 rows x 64
// columns and one wave computes it alone (no LDS, no barrier), with the
// operands read as 16-byte runs of 8 consecutive k -- exactly the MFMA
// fragment layout -- so the projection workgroups need no LDS and any wave
// count. Waves take tiles in row order from a shared counter; a wave that
// finishes a tile makes its stores visible at device scope (write-through
// `sc1` stores, then a wait for their completion) and adds one to the tile's
// row counter, ready[rt]. Row tile rt is complete when ready[rt] equals the
// number of column tiles. The recurrence reads Wx with `sc1` loads only after
// it has seen that count, so the rows reach it whichever XCD's L2 wrote them.
#pragma once

#include "frnn_device.h"
#include "frnn_kernels.h"

namespace frnn {

template <int MMA>
__device__ __forceinline__ void proj_load(Frag<MMA>& f, const unsigned short* p, bool ok) {
  const u16x8 v = ok ? *reinterpret_cast<const u16x8*>(p) : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
  if constexpr (MMA == MMA_BF16) f.v = __builtin_bit_cast(bf16x8, v);
  else f.v = __builtin_bit_cast(f16x8, v);
}

// One wave: take tiles until none are left. Every lane runs every iteration
// (the MFMAs need the whole wave); conditions on lanes are selects.
template <int MMA>
__device__ void proj_worker(const ProjArgs& pa) {
  static_assert(MMA != MMA_F32, "the projection workers are built for 16-bit operands");
  const int lane = threadIdx.x & 63, r16 = lane & 15, kq = lane >> 4;
  const int ntiles = pa.nrt * pa.nct;
  const long rows = (long)pa.B * pa.T;
  const unsigned short* x = static_cast<const unsigned short*>(pa.x);
  const unsigned short* w = static_cast<const unsigned short*>(pa.w);
  unsigned long long* wx = static_cast<unsigned long long*>(pa.wx);
  while (true) {
    // Every lane takes part in the grab (lane 0 adds 1, the others 0) and the
    // tile is lane 0's old value: a grab under `if (lane == 0)` at the head of
    // this loop was compiled into a loop whose exit only lane 0 could take,
    // the other lanes spinning on a stale tile index.
    const uint32_t old = __hip_atomic_fetch_add(pa.next, lane == 0 ? 1u : 0u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    const int tile = __builtin_amdgcn_readfirstlane((int)old);
    if (tile >= ntiles) break;
    const int rt = tile / pa.nct, ct = tile % pa.nct;
    // A operand: W rows (output columns) c = ct*64 + 16i + r16; B operand: x rows of m = rt*64 + 16j + r16
    const unsigned short* ap[4];
    const unsigned short* bp[4];
    bool av[4], bv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = ct * kProjCols + 16 * i + r16;
      av[i] = c < pa.ncols;
      ap[i] = w + (long)(av[i] ? c : 0) * pa.I + 8 * kq;
      const long m = (long)rt * kProjRows + 16 * i + r16;
      bv[i] = m < rows;
      const long mm = bv[i] ? m : 0;
      const long t = mm / pa.B, b = mm % pa.B;
      bp[i] = x + (b * pa.T + t) * pa.I + 8 * kq;
    }
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    Frag<MMA> fa0[4], fb0[4], fa1[4], fb1[4];
    auto load = [&](Frag<MMA>* fa, Frag<MMA>* fb, int k0) {
      // k beyond I: zeros, from an address kept inside the operand
      const bool kin = k0 + 8 * kq < pa.I;
      const int kk = kin ? k0 : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        proj_load<MMA>(fa[i], ap[i] + kk, kin && av[i]);
        proj_load<MMA>(fb[i], bp[i] + kk, kin && bv[i]);
      }
    };
    auto step = [&](const Frag<MMA>* fa, const Frag<MMA>* fb) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mma(fa[i], fb[j], acc[i][j]);
    };
    // two register sets: the loads of the next 32 k are in flight while the
    // current 32 run on the MFMA (k beyond I loads zeros)
    load(fa0, fb0, 0);
    for (int k0 = 0; k0 < pa.I; k0 += 64) {
      load(fa1, fb1, k0 + 32);
      step(fa0, fb0);
      load(fa0, fb0, k0 + 64);
      step(fa1, fb1);
    }
    // lane holds C^T[c = ct*64 + 16i + 4kq + 0..3][m = rt*64 + 16j + r16]:
    // four consecutive columns of one row, one 8-byte write-through store
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long m = (long)rt * kProjRows + 16 * j + r16;
      if (m >= rows) continue;
      const long t = m / pa.B, b = m % pa.B;
      const long row = (b * pa.T + t) * pa.ncols;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = ct * kProjCols + 16 * i + 4 * kq;
        if (c >= pa.ncols) continue;
        const unsigned long long v = (unsigned long long)op_bits<MMA>(acc[i][j][0]) |
                                     ((unsigned long long)op_bits<MMA>(acc[i][j][1]) << 16) |
                                     ((unsigned long long)op_bits<MMA>(acc[i][j][2]) << 32) |
                                     ((unsigned long long)op_bits<MMA>(acc[i][j][3]) << 48);
        __hip_atomic_store(wx + (row + c) / 4, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // the stores are complete (acknowledged at device scope) before the count
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_fetch_add(pa.ready + rt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace frnn

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
// Output rows are ordered by time: row m = t*B + b. Tiles are 128 output rows
// x 128 columns, taken in row order from a shared counter. A workgroup of four
// or more waves computes a tile together (proj_wg_worker): both operands are
// staged through LDS by LDS-DMA, two 64-deep k stages in flight, and each of
// four waves multiplies a 64 x 64 quarter. Where the recurrence's workgroups
// have fewer than four waves, each wave computes whole tiles alone
// (proj_wave_worker), as 64 x 64 quarters with operands read straight from
// memory. A finished tile's stores are made visible at device scope
// (write-through `sc1` stores, then a wait for their completion) before one
// is added to its row tile's counter, ready[rt]; row tile rt is complete when
// ready[rt] equals the number of column tiles. The recurrence reads Wx with
// device-coherent loads after it has seen that count, or with plain loads
// where the host found them safe (see fwd_io).
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

// Four FP32 accumulators of a 64 x 64 quarter stored as the output's 16-bit
// type: lane holds C^T[c = c0 + 16i + 4kq + 0..3][m = m0 + 16j + r16], four
// consecutive columns of one row, one 8-byte write-through store each.
template <int MMA>
__device__ __forceinline__ void proj_store(const ProjArgs& pa, const f32x4 (&acc)[4][4], int c0, long m0, int lane) {
  const int r16 = lane & 15, kq = lane >> 4;
  const long rows = (long)pa.B * pa.T;
  unsigned long long* wx = static_cast<unsigned long long*>(pa.wx);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const long m = m0 + 16 * j + r16;
    if (m >= rows) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = c0 + 16 * i + 4 * kq;
      if (c >= pa.ncols) continue;
      const unsigned long long v = (unsigned long long)op_bits<MMA>(acc[i][j][0]) |
                                   ((unsigned long long)op_bits<MMA>(acc[i][j][1]) << 16) |
                                   ((unsigned long long)op_bits<MMA>(acc[i][j][2]) << 32) |
                                   ((unsigned long long)op_bits<MMA>(acc[i][j][3]) << 48);
      __hip_atomic_store(wx + proj_wx_elem(pa, m, c) / 4, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Take the next tile: every lane of the calling wave takes part (lane 0 adds
// 1, the others 0) and the tile is lane 0's old value, uniform in a scalar
// register. (A grab under `if (lane == 0)` at the head of the tile loop was
// compiled into a loop that only lane 0 could leave, the other lanes spinning
// on a stale tile index.)
__device__ __forceinline__ int proj_grab(const ProjArgs& pa, int lane) {
  const uint32_t old = __hip_atomic_fetch_add(pa.next, lane == 0 ? 1u : 0u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_amdgcn_readfirstlane((int)old);
}

// One wave alone: whole tiles, each as four 64 x 64 quarters, operands read
// as 16-byte runs straight from memory (the MFMA fragment layout), the loads
// of the next 32 k in flight while the current 32 run on the MFMA.
template <int MMA>
__device__ void proj_wave_worker(const ProjArgs& pa) {
  static_assert(MMA != MMA_F32, "the projection workers are built for 16-bit operands");
  const int lane = threadIdx.x & 63, r16 = lane & 15, kq = lane >> 4;
  const int ntiles = pa.nrt * pa.nct;
  const unsigned short* w = static_cast<const unsigned short*>(pa.w);
  while (true) {
    const int tile = proj_grab(pa, lane);
    if (tile >= ntiles) break;
    const int rt = tile / pa.nct, ct = tile % pa.nct;
    for (int quarter = 0; quarter < 4; ++quarter) {
      const int c0 = ct * kProjCols + 64 * (quarter & 1);
      const long m0 = (long)rt * kProjRows + 64 * (quarter >> 1);
      const unsigned short* x = static_cast<const unsigned short*>(pa.x);
      const unsigned short* ap[4];
      const unsigned short* bp[4];
      bool av[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        av[i] = c0 + 16 * i + r16 < pa.ncols;
        ap[i] = w + proj_w_row(pa, c0 + 16 * i + r16);
        bp[i] = x + proj_x_row(pa, m0 + 16 * i + r16);
      }
      f32x4 acc[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      Frag<MMA> fa0[4], fb0[4], fa1[4], fb1[4];
      auto load = [&](Frag<MMA>* fa, Frag<MMA>* fb, int k0) {
        // k beyond I: zeros (the address stays inside the operand)
        const bool kin = k0 + 8 * kq < pa.I;
        const int k8 = proj_k8(pa, k0 + 8 * kq);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          proj_load<MMA>(fa[i], ap[i] + k8, kin && av[i]);
          proj_load<MMA>(fb[i], bp[i] + k8, kin);
        }
      };
      auto step = [&](const Frag<MMA>* fa, const Frag<MMA>* fb) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mma(fa[i], fb[j], acc[i][j]);
      };
      load(fa0, fb0, 0);
      for (int k0 = 0; k0 < pa.I; k0 += 64) {
        load(fa1, fb1, k0 + 32);
        step(fa0, fb0);
        load(fa0, fb0, k0 + 64);
        step(fa1, fb1);
      }
      proj_store<MMA>(pa, acc, c0, m0, lane);
    }
    // the stores are complete (acknowledged at device scope) before the count
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_fetch_add(pa.ready + rt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// LDS bytes of proj_wg_worker: two stages of a 128 x 64 tile of each operand, and the tile slots.
constexpr int kProjStage = 2 * 128 * 128;  // bytes per stage: W rows, then x rows (128 B of k per row)
constexpr int kProjLds = 2 * kProjStage + 16;

// LDS position of (row r, 16-byte chunk q of its 64 k) in a 128-row operand
// tile: the chunk index is XORed with (r / 2) % 8, so the 16 rows one
// fragment read touches in a pass (rows r..r+15, one chunk) hit 16 distinct
// 16-byte bank groups.
__device__ __forceinline__ int proj_lds_off(int r, int q) { return r * 128 + ((q ^ (r >> 1)) & 7) * 16; }

// Four waves together (waves beyond four leave at once: a barrier waits only
// for the waves still running): one 128 x 128 tile per grab, k in stages of 64.
template <int MMA>
__device__ void proj_wg_worker(const ProjArgs& pa, char* lds) {
  static_assert(MMA != MMA_F32, "the projection workers are built for 16-bit operands");
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (wv >= 4) return;
  const int lane = threadIdx.x & 63, r16 = lane & 15, kq = lane >> 4;
  const int ntiles = pa.nrt * pa.nct;
  const int nk = (pa.I + 63) / 64;
  int* slot = reinterpret_cast<int*>(lds + 2 * kProjStage);  // the grabbed tile, read after a barrier
  const unsigned short* w = static_cast<const unsigned short*>(pa.w);
  // DMA: wave wv fills rows wv*32 .. wv*32+31 of each operand, eight rows per
  // instruction; lane L of instruction j: row wv*32 + 8j + L/8, its chunk at
  // LDS position L%8 (which holds logical chunk (L%8) ^ ((row/2)%8)).
  const int lrow = lane >> 3, lpos = lane & 7;
  // quarter of this wave: columns 64*(wv&1).., rows 64*(wv>>1)..
  const int qc = 64 * (wv & 1), qm = 64 * (wv >> 1);
  int iter = 0;
  while (true) {
    if (wv == 0) {
      const int t = proj_grab(pa, lane);
      if (lane == 0) slot[iter & 1] = t;
    }
    lds_barrier();
    const int tile = __builtin_amdgcn_readfirstlane(slot[iter & 1]);
    ++iter;
    if (tile >= ntiles) break;
    const int rt = tile / pa.nct, ct = tile % pa.nct;
    const int c0 = ct * kProjCols;
    const long m0 = (long)rt * kProjRows;
    const unsigned short* x = static_cast<const unsigned short*>(pa.x);
    const unsigned short* asrc[4];
    const unsigned short* bsrc[4];
    int qlog[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wv * 32 + 8 * j + lrow;
      qlog[j] = (lpos ^ (r >> 1)) & 7;
      asrc[j] = w + proj_w_row(pa, c0 + r);
      bsrc[j] = x + proj_x_row(pa, m0 + r);
    }
    auto issue = [&](int k0) {
      char* st = lds + (k0 / 64 & 1) * kProjStage;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k8 = proj_k8(pa, k0 + 8 * qlog[j]);
        __builtin_amdgcn_global_load_lds(asrc[j] + k8,
                                         (__attribute__((address_space(3))) void*)(st + (wv * 32 + 8 * j) * 128),
                                         16, 0, 0);
        __builtin_amdgcn_global_load_lds(bsrc[j] + k8,
                                         (__attribute__((address_space(3))) void*)(st + 128 * 128 + (wv * 32 + 8 * j) * 128),
                                         16, 0, 0);
      }
    };
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    issue(0);
    for (int ks = 0; ks < nk; ++ks) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();  // stage ks landed for every wave; every wave is done with stage ks-1
      if (ks + 1 < nk) issue(64 * (ks + 1));
      const char* st = lds + (ks & 1) * kProjStage;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int q = 4 * s + kq;
        const bool kin = 64 * ks + 8 * q < pa.I;
        Frag<MMA> fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          u16x8 va = *reinterpret_cast<const u16x8*>(st + proj_lds_off(qc + 16 * i + r16, q));
          u16x8 vb = *reinterpret_cast<const u16x8*>(st + 128 * 128 + proj_lds_off(qm + 16 * i + r16, q));
          if (!kin) va = vb = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
          if constexpr (MMA == MMA_BF16) {
            fa[i].v = __builtin_bit_cast(bf16x8, va);
            fb[i].v = __builtin_bit_cast(bf16x8, vb);
          } else {
            fa[i].v = __builtin_bit_cast(f16x8, va);
            fb[i].v = __builtin_bit_cast(f16x8, vb);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mma(fa[i], fb[j], acc[i][j]);
      }
    }
    proj_store<MMA>(pa, acc, c0 + qc, m0 + qm, lane);
    // every wave's stores complete (acknowledged at device scope), then one count
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    if (wv == 0 && lane == 0) __hip_atomic_fetch_add(pa.ready + rt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace frnn

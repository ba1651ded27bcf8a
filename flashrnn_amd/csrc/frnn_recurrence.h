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
// elements e = s*KS*64 + kw*64 + lane; I/O lane l serves e = io_elem(l, i)
// (frnn_plan.h).
#pragma once

#include "frnn_cells.h"
#include "frnn_device.h"
#include "frnn_kernels.h"
#include "frnn_plan.h"
#include "frnn_proj.h"

namespace frnn {

constexpr int kFwdRing = 2;   // raw Wx slots in LDS (DMA targets)
constexpr int kFwdXf = 3;     // converted (FP32) Wx slots in LDS (what the owners read)
constexpr int kGateBatch = 4;  // projection-readiness counters read per poll
constexpr int kFwdAhead = 3;  // steps a Wx load goes out ahead of its use

// Backward input pipeline: the I/O wave keeps kBwdRegs iterations of loads in
// flight in registers and stages inputs into kBwdStage LDS slots, two
// iterations ahead of their use, so the owners can read an iteration's inputs
// during the previous iteration's poll.
constexpr int kBwdRegs = 2;
constexpr int kBwdStage = 3;

// LDS layout of a team:
//   forward : red  [2][KS][NB][272 slots][4 gates]        MFMA partial sums; slot
//                  red_slot(lane*4 + reg): one spare slot per 16, so both the
//                  16-byte writes (lane-major) and the owners' reads (element-
//                  major) hit 16 distinct bank groups per 16 lanes
//             xring[slot][gate][64 chunks][16 bytes]       raw Wx of the next steps
//                  (chunk = row * 4 + quad: FP32 units 4*quad..+3; BF16 units
//                   4*quad..+7 in the even quads, odd quads unused)
//             ost  [2][value][NE]                         states + saved values (FP32),
//                  value-major so the drain reads 4 elements per 16-byte read
//             xf   [slot][gate][NE]                       Wx of a step in FP32,
//                  converted from the raw slot by the I/O wave
//   backward: red  [2][NB][KS][304]                       partial R^T dG at
//                  red_idx(lane*4 + reg): 16 spare floats per 64, so the
//                  16-byte writes and the owners' scalar reads are conflict-free
//             iring[3][S + NSAVE][NE]                     state cotangents + saved values,
//                  value-major: the I/O wave writes four elements of a value
//                  per 16-byte write (lane-contiguous, no bank conflicts)
//             ost  [2][4][NE]                             dWx (+ GRU candidate cotangent),
//                  value-major likewise
template <int CELL, int NB>
struct Lds {
  static constexpr int NE = NB * 256;
  static constexpr int GR = CellShape<CELL>::GR, GW = CellShape<CELL>::GW, S = CellShape<CELL>::S;
  static constexpr int NSAVE = Cell<CELL>::NSAVE;
  static constexpr int NOB = 4;                              // backward outputs per element, padded
  // floats per team
  static constexpr int NV = S + NSAVE;                      // staged values per element (forward)
  static constexpr int RING = GW * 64 * 4;                   // floats per Wx ring slot
  static constexpr int RED_F = 272 * 4;  // floats per (wave, batch tile), forward partials
  // floats per (batch tile, wave), backward partials: 304 used, padded to a
  // multiple of 64 floats so the owners' KS reads of one element, RED_B apart,
  // pair into ds_read2st64 (C2 backward 1.545 -> 1.53 ms)
  static constexpr int RED_B = 320;
  static constexpr int XF = GW * NE;                         // floats per converted Wx slot
  __host__ __device__ static constexpr long fwd(int KS) {
    return 2L * KS * NB * RED_F + (long)kFwdRing * RING + 2L * NV * NE + (long)kFwdXf * XF;
  }
  __host__ __device__ static constexpr long bwd(int KS) {
    return 2L * NB * KS * RED_B + (long)kBwdStage * NE * NV + 2L * NE * NOB + 16;  // + the owners' step flags
  }
};

// Tag a poll waits for: the step's, or (kFlagUnready, failure-handling tests)
// 3, which is never written.
__device__ __forceinline__ uint32_t ptag(const Plan& p, int step) {
  return (p.flags & kFlagUnready) ? 3u : step_tag(step);
}

// Padded positions of the partial-sum layouts (see Lds).
__device__ __forceinline__ int red_slot(int s) { return s + (s >> 4); }
__device__ __forceinline__ int red_idx(int s) { return s + (s >> 6) * 16; }

struct Team {
  int lane, w, row, kq;  // lane in wave, wave in workgroup, lane%16, lane/16
  int team, kw;          // hidden tile (team) of this wave, its contraction split (kw == KS: I/O wave)
  int group, member, n, slab, dt, wgi;
};

// XCD-local exchange: the workgroup claims the next free slot of the XCD it
// runs on (read from the hardware), so every group is XCD-local whatever order
// the dispatcher hands workgroups to XCDs in. A launch's grid holds the same
// number of slots on every XCD; a workgroup beyond them (an uneven dispatch)
// raises the placement status and leaves, and its partners time out.
// The claim is broadcast through the first word of the kernel's dynamic LDS
// (a static __shared__ variable would shift the dynamic area off its 16-byte
// alignment), which is free again after the second barrier.
__device__ __forceinline__ bool team_setup(const Plan& p, Team& tm, uint32_t* claim, uint32_t* status, int KS,
                                           float* lds) {
  int wg = blockIdx.x, xcd = 0;
  if (!(p.flags & 2)) {
    volatile uint32_t* s_slot = reinterpret_cast<volatile uint32_t*>(lds);
    xcd = (int)(xcc_id() & 15u);
    if (threadIdx.x == 0)
      *s_slot = xcd < kXcds ? __hip_atomic_fetch_add(claim + (long)p.g0 * kXcds + xcd, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)
                            : 0xffffffffu;
    __syncthreads();
    const uint32_t slot = *s_slot;
    __syncthreads();
    if (slot >= (uint32_t)((p.grid - scout_blocks(p)) / kXcds)) {
      if (threadIdx.x == 0) raise_status(status, ST_PLACEMENT);
      return false;  // the whole workgroup leaves together
    }
    wg = (int)slot;
  }
  if (!wg_decode(p, wg, xcd, &tm.group, &tm.member)) return false;
  tm.lane = threadIdx.x & 63;
  tm.w = threadIdx.x >> 6;
  tm.team = tm.w / (KS + 1);
  tm.kw = tm.w % (KS + 1);
  tm.row = tm.lane & 15;
  tm.kq = tm.lane >> 4;
  tm.n = tm.group / p.nslab;
  tm.slab = tm.group % p.nslab;
  tm.dt = tm.member * p.NDT + tm.team;
  tm.wgi = tm.group * p.wpg + tm.member;
  return true;
}

// A scout claims the next scout slot of its XCD (counters after the members')
// and takes the group of that slot; a slot beyond the XCD's groups leaves.
__device__ __forceinline__ bool scout_setup(const Plan& p, Team& tm, uint32_t* claim, float* lds) {
  volatile uint32_t* s_slot = reinterpret_cast<volatile uint32_t*>(lds);
  const int xcd = (int)(xcc_id() & 15u);
  if (threadIdx.x == 0)
    *s_slot = xcd < kXcds ? __hip_atomic_fetch_add(claim + ((long)p.ngroups + p.g0) * kXcds + xcd, 1u,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : 0xffffffffu;
  __syncthreads();
  const uint32_t slot = *s_slot;
  __syncthreads();
  const int nsc = p.nscout > 1 ? p.nscout : 1;
  if (slot >= (uint32_t)((p.gcount + kXcds - 1) / kXcds * nsc)) return false;
  const int local = (int)(slot / nsc) * kXcds + xcd;
  if (local >= p.gcount) return false;
  tm.group = p.g0 + local;
  tm.member = (int)(slot % nsc);  // this scout's share of the group's touches
  tm.n = tm.group / p.nslab;
  tm.slab = tm.group % p.nslab;
  return true;
}

// Element e of the team -> hidden unit d, slab row bl, batch row b.
typedef ElemPos Elem;
__device__ __forceinline__ Elem elem_of(const Plan& p, const Team& tm, int e) { return elem_pos(p, tm.slab, tm.dt, e); }
// Owner slot i (s * KS * 64 + compute wave * 64 + lane) -> element in the
// one-tile forward: the 16 rows of a batch tile are dealt to the slots'
// 16-lane quarters round-robin (quarter q takes row 4 (q % 4) + q / 4: the
// owner waves of four compute waves hold rows kw, kw + 4, kw + 8, kw + 12), so
// a slab with fewer than 16 real rows still gives every owner wave a share of
// the real work (measured, LSTM T1024 N3 D256 forward: B8 1.28 -> 1.25 ms, B4
// 1.30 -> 1.24, B16 1.41 -> 1.38; the backward, the two-tile forward and the
// sLSTM forward (C4 B16 D192 2.81 -> 2.93 ms: more staged values, whose LDS
// writes the round-robin rows spread over fewer banks) keep slot order).
__device__ __forceinline__ int owner_elem(int i) {
  const int q = (i >> 4) & 15;
  return (i & ~255) | ((((q & 3) << 2) | (q >> 2)) << 4) | (i & 15);
}
// Position of element e in the MFMA output layout of its batch tile: lane
// (dd/4)*16 + row, register dd%4 (dd = hidden unit in the tile), as lane*4 + reg.
__device__ __forceinline__ int mfma_pos(int e) {
  const int r = e & 255, dd = r & 15, bb = r >> 4;
  return ((dd >> 2) * 16 + bb) * 4 + (dd & 3);
}


// Phase profile of every wave of workgroup 0 (8 words per wave). Compute
// waves: cycles in [0] exchange wait, [1] MFMA + LDS partials, [2] barrier,
// [3] owners' cell work (backward: pointwise), [4] exchange polls, [5] steps,
// [6] backward: reduction of the partial cotangents. I/O waves: [0] ring fill
// (waits for its loads), [1] load issue, [2] barrier, [3] output drain, [5] steps.
//
// With profiling on, every wave of every workgroup also keeps a timeline of
// steps kTraceT0 .. kTraceT0+7: eight stamps per step from the chip-wide
// 100 MHz clock (s_memrealtime), lane `slot` holding stamp `slot`, written
// after the loop to trace[(workgroup * 16 + wave) * 64 + lane].
constexpr int kTraceT0 = 64;
struct Prof {
  unsigned long long acc[8];
  unsigned long long t;
  unsigned long long tv;
  bool on, tr;
  __device__ __forceinline__ void init(bool enable, bool trace = false) {
    on = enable;
    tr = trace;
    tv = 0;
    for (int i = 0; i < 8; ++i) acc[i] = 0;
    t = on ? clock64() : 0;
  }
  // Record a value (not a time) in slot k of a traced step.
  __device__ __forceinline__ void put(int step, int k, unsigned long long v) {
    if (!tr) return;
    const int slot = (step - kTraceT0) * 8 + k;
    if (slot < 0 || slot >= 64) return;
    if ((int)(threadIdx.x & 63) == slot) tv = v;
  }
  __device__ __forceinline__ void stamp(int step, int k) {
    if (!tr) return;
    const int slot = (step - kTraceT0) * 8 + k;
    if (slot < 0 || slot >= 64) return;
    const unsigned long long now = __builtin_amdgcn_s_memrealtime();
    if ((int)(threadIdx.x & 63) == slot) tv = now;
  }
  // Slot 7 (stamp 7 of the first traced step, never stamped) carries the
  // workgroup's (group, member) as group * 65536 + member.
  __device__ __forceinline__ void flush_trace(unsigned long long* trace, const Team& tm) {
    if ((threadIdx.x & 63) == 7) tv = (unsigned long long)tm.group * 65536ull + (unsigned long long)tm.member;
    if (tr && blockIdx.x < 128) trace[(blockIdx.x * 16 + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63)] = tv;
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
      for (int i = 0; i < 8; ++i) out[(threadIdx.x >> 6) * 8 + i] = acc[i];
  }
};


// Work a gather runs once, right after it issues its first poll's loads (the
// wait for them then overlaps it).
struct NoWork {
  __device__ __forceinline__ void operator()() const {}
};

// Runs a wave keeps in flight at most (8 BF16 runs or 4 FP32 runs: 64
// registers; 4 runs in two-tile workgroups, whose resident slice is larger);
// a longer contraction range is polled chunk by chunk, which bounds the
// registers of the in-flight loads.
template <int MMA, int NDT> struct PollChunk {
  static constexpr int value = (MMA != MMA_F32 && NDT == 1) ? 8 : 4;
};

// Poll the exchange and run the step's product on it, fused. Every 8-word run
// of this wave's contraction range is loaded at once; as each arrives it is
// unpacked, its tags checked, and its MFMAs issued into the caller's
// accumulators, so the products overlap the tail of the loads. If any tag is
// stale the accumulators are cleared and the poll repeats. Runs of padded batch
// rows are not read (they contribute zero). zero() clears the accumulators,
// prod(bt, j, frag) adds run j of batch tile bt. Returns the number of polls.
//
// Ranges of more than PollChunk runs are polled in chunks: each chunk is
// polled until all of its tags are fresh and only then multiplied, so a
// stale chunk never has to be taken back out of the accumulators.
template <int MMA, int NDT, int NB, int NF, bool SPLIT = false, bool SPEC = true, bool PIPE = false, typename Zero,
          typename Prod, typename Between = NoWork>
__device__ __forceinline__ uint32_t gather_mma(const Xchg& x, const int (&word)[NB][NF], const bool (&bval)[NB],
                                               int off, int cstride, int nf, uint32_t tag, uint32_t* status, uint32_t spin_limit,
                                               bool& abort, Zero zero, Prod prod, Between between = Between{}) {
  bool first = true;
  using Op = Operand<MMA, SPLIT>;
  uint32_t spins = 0;
  // A wave with no k-tiles (more compute waves than k-tiles) polls nothing but
  // still does its between-work. Handled here where each wave has at most one
  // k-tile (NF == 1); the GRU's backward at D = 32 (three k-tiles over four
  // waves, NF = 3) keeps such a wave out of the gather itself.
  if constexpr (NF == 1) {
    if (nf <= 0) {
      zero();
      between();
      return 0;
    }
  }
  if constexpr (NF <= PollChunk<MMA, NDT>::value && SPEC) {
    while (true) {
      zero();
      if (abort) return spins;
      Run<MMA> r[NB][NF];
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int j = 0; j < NF; ++j) {
          r[bt][j].zero();
          if (j < nf && bval[bt]) xload<MMA>(x, word[bt][j] + off, cstride, r[bt][j]);
        }
      if (first) {
        between();
        first = false;
      }
      // Branch-free from here on: the MFMAs read operands across lanes and must
      // run with the whole wave active, so lane-dependent conditions are selects.
      bool ok = true;
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int j = 0; j < NF; ++j)
          if (j < nf) {
            Op o;
            const bool fresh = o.unpack(r[bt][j], tag);
            ok &= fresh || !bval[bt];
            o.keep(bval[bt]);
            o.apply([&](const Frag<MMA>& f, int part) { prod(bt, j, f, part); });
          }
      ++spins;
      if (__all(ok)) return spins;
      if (spins >= spin_limit) {
        raise_status(status, ST_TIMEOUT);
        abort = true;
      } else if ((spins & 63u) == 0 && load_status(status) != 0) {
        abort = true;
      }
    }
  } else if constexpr (PIPE) {
    constexpr int CH = NF < PollChunk<MMA, NDT>::value ? NF : PollChunk<MMA, NDT>::value;
    zero();
    // PIPE: the next chunk's loads go out as soon as the current chunk is
    // fresh and unpacked, before its products, so its round trip overlaps them
    // (the unpacked chunk costs registers: used where they fit).
    Run<MMA> r[NB][CH];
    auto issue = [&](int c0) {
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int jj = 0; jj < CH; ++jj) {
          r[bt][jj].zero();
          if (c0 + jj < NF && c0 + jj < nf && bval[bt]) xload<MMA>(x, word[bt][c0 + jj < NF ? c0 + jj : 0] + off, cstride, r[bt][jj]);
        }
    };
    issue(0);
    between();
#pragma unroll
    for (int c0 = 0; c0 < NF; c0 += CH) {
      if (c0 >= nf) break;
      while (true) {
        if (abort) return spins;
        bool ok = true;
#pragma unroll
        for (int bt = 0; bt < NB; ++bt)
#pragma unroll
          for (int jj = 0; jj < CH; ++jj)
            if (c0 + jj < NF && c0 + jj < nf) ok &= Op::fresh(r[bt][jj], tag) || !bval[bt];
        ++spins;
        if (__all(ok)) break;
        if (spins >= spin_limit) {
          raise_status(status, ST_TIMEOUT);
          abort = true;
        } else if ((spins & 63u) == 0 && load_status(status) != 0) {
          abort = true;
        }
        issue(c0);
      }
      Op o[NB][CH];
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int jj = 0; jj < CH; ++jj) {
          o[bt][jj].unpack(r[bt][jj], tag);
          o[bt][jj].keep(bval[bt]);
        }
      if (c0 + CH < NF && c0 + CH < nf) issue(c0 + CH);
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int jj = 0; jj < CH; ++jj)
          if (c0 + jj < NF && c0 + jj < nf)
            o[bt][jj].apply([&](const Frag<MMA>& f, int part) { prod(bt, c0 + jj, f, part); });
    }
    return spins;
  } else {
    constexpr int CH = NF < PollChunk<MMA, NDT>::value ? NF : PollChunk<MMA, NDT>::value;
    zero();
#pragma unroll
    for (int c0 = 0; c0 < NF; c0 += CH) {
      if (c0 >= nf) break;
      while (true) {
        if (abort) return spins;
        Run<MMA> r[NB][CH];
#pragma unroll
        for (int bt = 0; bt < NB; ++bt)
#pragma unroll
          for (int jj = 0; jj < CH; ++jj) {
            r[bt][jj].zero();
            if (c0 + jj < NF && c0 + jj < nf && bval[bt]) xload<MMA>(x, word[bt][c0 + jj < NF ? c0 + jj : 0] + off, cstride, r[bt][jj]);
          }
        if (first) {
          between();
          first = false;
        }
        bool ok = true;
#pragma unroll
        for (int bt = 0; bt < NB; ++bt)
#pragma unroll
          for (int jj = 0; jj < CH; ++jj)
            if (c0 + jj < NF && c0 + jj < nf) ok &= Op::fresh(r[bt][jj], tag) || !bval[bt];
        ++spins;
        if (__all(ok)) {
#pragma unroll
          for (int bt = 0; bt < NB; ++bt)
#pragma unroll
            for (int jj = 0; jj < CH; ++jj)
              if (c0 + jj < NF && c0 + jj < nf) {
                Op o;
                o.unpack(r[bt][jj], tag);
                o.keep(bval[bt]);
                o.apply([&](const Frag<MMA>& f, int part) { prod(bt, c0 + jj, f, part); });
              }
          break;
        }
        if (spins >= spin_limit) {
          raise_status(status, ST_TIMEOUT);
          abort = true;
        } else if ((spins & 63u) == 0 && load_status(status) != 0) {
          abort = true;
        }
      }
    }
    return spins;
  }
}

// Paired variant for slabs with at most 8 real batch rows (one 16-row tile):
// the upper half of each 16-lane row (padding columns of the MFMA operand)
// polls the odd k-tile of each pair for the same batch row, so a lane issues
// half the loads; the odd tile then moves down 8 lanes (DPP) and the upper
// lanes contribute zero. word[j] is the run of k-tile j for batch row lane % 8.
// Long ranges are polled in chunks of PollChunk pairs, as in gather_mma.
//
// Split words (SPLIT) fill the padding columns instead: the even tile's
// product takes hi in columns 0-7 and lo in columns 8-15 of one B operand, the
// odd tile's likewise, so a pair costs two MFMAs, not four (one DPP rotation
// trades the lower lanes' lo for the upper lanes' hi). Columns 0-7 of the
// accumulators then hold the hi products and columns 8-15 the lo products of
// the same batch rows; the caller adds column c + 8 into column c
// (fold_cols8) before it reads them.
template <int MMA, int NDT, int NF, bool SPLIT = false, bool SPEC = true, typename Zero, typename Prod,
          typename Between = NoWork>
__device__ __forceinline__ uint32_t gather_pair_mma(const Xchg& x, const int (&word)[NF], bool bv, int off, int cstride, int nf,
                                                    uint32_t tag, uint32_t* status, uint32_t spin_limit, bool& abort,
                                                    Zero zero, Prod prod, Between between = Between{}) {
  bool first = true;
  using Op = Operand<MMA, SPLIT>;
  constexpr int NP = (NF + 1) / 2;
  constexpr int CH = NP <= PollChunk<MMA, NDT>::value ? NP : PollChunk<MMA, NDT>::value;
  // speculative: one chunk, multiplied while its tags are checked; otherwise
  // each chunk is multiplied once all of its tags are fresh
  constexpr bool kSpec = SPEC && NP <= PollChunk<MMA, NDT>::value;
  // A wave with no k-tiles polls nothing but still does its between-work (see
  // gather_mma for NF > 1).
  if constexpr (NF == 1) {
    if (nf <= 0) {
      zero();
      between();
      return 0;
    }
  }
  const int hi = (threadIdx.x >> 3) & 1;  // lane % 16 >= 8
  // the pair's products: the even tile in place, the odd one moved down 8 lanes
  auto pair_prod = [&](Op o, int i) {
    if constexpr (SPLIT) {
      // lower lanes hold (hi, lo) of the even tile, upper lanes those of the odd tile
      const Frag<MMA> got = frag_rot8(frag_sel<MMA>(hi, o.hi, o.lo));  // lower: hi_odd, upper: lo_even
      prod(0, 2 * i, frag_sel<MMA>(hi, got, o.hi), 0);                   // [hi_even | lo_even]
      if (2 * i + 1 < nf) prod(0, 2 * i + 1, frag_sel<MMA>(hi, o.lo, got), 0);  // [hi_odd | lo_odd]
    } else {
      const Op odd = o.rot8();
      o.keep(!hi);
      o.apply([&](const Frag<MMA>& f, int part) { prod(0, 2 * i, f, part); });
      if (2 * i + 1 < nf) {
        Op od = odd;
        od.keep(!hi);
        od.apply([&](const Frag<MMA>& f, int part) { prod(0, 2 * i + 1, f, part); });
      }
    }
  };
  uint32_t spins = 0;
  zero();
#pragma unroll
  for (int i0 = 0; i0 < NP; i0 += CH) {
    if (2 * i0 >= nf) break;
    while (true) {
      if constexpr (kSpec) zero();
      if (abort) return spins;
      Run<MMA> r[CH];
#pragma unroll
      for (int ii = 0; ii < CH; ++ii) {
        const int i = i0 + ii;
        r[ii].zero();
        if (i < NP && 2 * i + hi < nf && bv) xload<MMA>(x, word[i < NP ? 2 * i + hi : 0] + off, cstride, r[ii]);
      }
      if (first) {
        between();
        first = false;
      }
      // Branch-free from here on (cross-lane DPP and MFMA need the whole wave).
      bool ok = true;
      if constexpr (kSpec) {
#pragma unroll
        for (int ii = 0; ii < CH; ++ii) {
          const int i = i0 + ii;
          if (2 * i >= nf) continue;
          const bool v = 2 * i + hi < nf && bv;
          Op o;
          const bool fresh = o.unpack(r[ii], tag);
          ok &= fresh || !v;
          o.keep(v);
          pair_prod(o, i);
        }
      } else {
#pragma unroll
        for (int ii = 0; ii < CH; ++ii) {
          const int i = i0 + ii;
          if (i >= NP || 2 * i >= nf) continue;
          const bool v = 2 * i + hi < nf && bv;
          ok &= Op::fresh(r[ii], tag) || !v;
        }
      }
      ++spins;
      if (__all(ok)) {
        if constexpr (!kSpec) {
#pragma unroll
          for (int ii = 0; ii < CH; ++ii) {
            const int i = i0 + ii;
            if (i >= NP || 2 * i >= nf) continue;
            const bool v = 2 * i + hi < nf && bv;
            Op o;
            o.unpack(r[ii], tag);
            o.keep(v);
            pair_prod(o, i);
          }
        }
        break;
      }
      if (spins >= spin_limit) {
        raise_status(status, ST_TIMEOUT);
        abort = true;
      } else if ((spins & 63u) == 0 && load_status(status) != 0) {
        abort = true;
      }
    }
  }
  return spins;
}

// Accumulator lane l, register i holds column l % 16: add column c + 8 into
// column c (lanes l and l ^ 8 of each 16-lane row; both get the sum).
// (All four rotations read the unmodified accumulator and go through one
// vector: an element-by-element read-modify-write of the accumulator was
// compiled into rotations of the already-updated element 0 for elements 1-3.)
__device__ __forceinline__ f32x4 fold_cols8(f32x4 v) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 r = __builtin_bit_cast(i32x4, v);
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = rot8(r[i]);
  return v + __builtin_bit_cast(f32x4, r);
}

// Element-size class of an I/O wave: 0 = 16-bit tensors and states, 1 = 16-bit
// tensors (Wx, dWx) with FP32 states (snapshot), 2 = FP32 tensors and states.
__host__ __device__ __forceinline__ int io_sizes(int dt_io, int dt_out) {
  return dt_io == DT_F32 ? 2 : (dt_out == DT_F32 ? 1 : 0);
}
// Bytes of a saved-for-backward value: FP16 under the 16-bit operand policies
// (LSTM, GRU, Elman), FP32 for FP32 operands and for the sLSTM (the host plan's
// dt_save says the same).
template <int CELL, int MMA> struct SaveSize {
  static constexpr int value = (MMA != MMA_F32 && CELL != CELL_SLSTM) ? 2 : 4;
};

// ====================================================================== forward
// I/O lane l serves the elements io_elem(l, i) = 256*(i/4) + 4*l + i%4: four
// consecutive hidden units of one batch row, so every global access is one
// 8/16-byte vector access and every LDS access one 16-byte access.

// I/O wave of a team. Wx of step u is loaded straight into raw slot u % 2 by
// LDS-DMA (global_load_lds: no registers in flight), three steps ahead; two
// steps ahead of its use the wave converts it to FP32 in slot u % 3 of the
// area the owners read (so the runtime dtype is off their critical path).
// After barrier t it also drains step t-1's outputs from the staging area.
// Per step the wave issues the same loads and stores in the same order, so the
// count of operations issued after a step's loads is a constant in the steady
// state. Padding batch rows are neither loaded nor stored (their converted
// values are never used).
//
// XS, OS, SS: element sizes (2 or 4 bytes) of Wx, of the state output and of
// the saved values, fixed at compile time; BF16 vs FP16 is a branch-free
// select. This wave sits close to the step's critical path: each of its LDS
// bursts (all reads, then all writes or stores) issues without waiting
// between the accesses.
template <int CELL, int MMA, int NB, int XS, int OS, int SS, bool PROJ>
__device__ void fwd_io(const FwdArgs& a, const Team& tm, float* xring, float* ost, float* xf) {
  static_assert(NB == 1, "one 16-row batch tile per group");
  using CS = CellShape<CELL>;
  constexpr int GW = CS::GW, S = CS::S, NE = NB * 256, P = kFwdAhead;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NV = Lds<CELL, NB>::NV, RING = Lds<CELL, NB>::RING;
  const Plan& p = a.p;
  const int T = p.T, N = p.N, D = p.D, B = p.B, TT = p.Ttot, t0 = p.t0;
  const bool training = (p.flags & 1) != 0;
  const bool xf16 = p.dt_io == DT_F16, of16 = p.dt_out == DT_F16, sf16 = p.dt_save == DT_F16;
  // output policy: all S states, the hidden state only, or the sequence's last hidden state only
  const int mode = (p.flags & kFlagOutLast) ? 2 : ((p.flags & kFlagOutHidden) ? 1 : 0);
  const int nst = mode == 0 ? S : 1;
  const long wx_t = (long)GW * N * D;
  // loads: lane -> (row, quad); 16-bit chunks hold 8 units, so odd quads idle
  const int lrow = tm.lane >> 2, lquad = tm.lane & 3;
  bool lval;
  const long lbase = wx_dma_index(p, tm.slab, tm.n, tm.dt, tm.lane, 0, 0, XS, &lval);  // + u * wx_t + g * N * D
  // Projection-gated launches (the launch also runs the input projection, see
  // frnn_proj.h): before the loads of step u, wait until every row tile that
  // step reads is complete. The loads are device-coherent (sc1) unless the
  // host found them safe as plain, L2-cached loads (proj.plain): workers only
  // on XCDs without groups, and Wx rows that are whole 128-byte lines, so no
  // line this XCD's L2 fetches holds bytes of a row that is not yet complete
  // (the kernel's start leaves no stale line in it). The wait walks the row
  // tiles in order and remembers how far it got. A wait past the spin limit
  // raises the timeout status and stops waiting (every wave still runs to the end).
  int ready_rt = 0;
  bool gave_up = false;
  auto gate = [&](int u) {
    if constexpr (PROJ) {
      const int need = proj_last_row_tile(u, B);
      uint32_t spins = 0;
      while (ready_rt <= need && !gave_up) {
        // four counters per poll (each poll waits for this wave's earlier
        // loads and stores): the wait passes every complete row tile in a row
        uint32_t v[kGateBatch];
#pragma unroll
        for (int k = 0; k < kGateBatch; ++k)
          v[k] = ready_rt + k < a.proj.nrt
                     ? __hip_atomic_load(a.proj.ready + ready_rt + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0u;
        const int before = ready_rt;
#pragma unroll
        for (int k = 0; k < kGateBatch; ++k)
          if (ready_rt == before + k && v[k] >= (uint32_t)a.proj.nct) ++ready_rt;
        if (ready_rt > before) continue;
        __builtin_amdgcn_s_sleep(2);
        if (++spins >= a.spin_limit) {
          raise_status(a.status, ST_TIMEOUT);
          gave_up = true;
        } else if ((spins & 255u) == 0 && load_status(a.status) != 0) {
          gave_up = true;
        }
      }
    }
  };
  auto load_wx = [&](int u) {
    gate(u);
    float* slot = xring + (long)(u % kFwdRing) * RING;
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const char* src = static_cast<const char*>(a.wx) + (lbase + (long)u * wx_t + (long)g * N * D) * XS;
      if (lval) {
        auto dst = (__attribute__((address_space(3))) void*)(slot + g * 256);
        if (PROJ && !a.proj.plain) __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 16);
        else __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
      }
    }
  };
  // stores: lane -> elements e0 .. e0+3 (four units of one row), from base
  // offsets that advance by a constant per step
  const int e0 = io_elem(tm.lane, 0);
  const Elem el = elem_of(p, tm, e0);
  long st_off[S];
#pragma unroll
  for (int k = 0; k < S; ++k) st_off[k] = state_index(p, k, el.b, 0, tm.n, el.d);
  const long st_step = (long)N * D;  // state_index per window step
  const long sv_off = save_index(p, NE, 0, tm.wgi, 0, tm.team, e0);
  const long sv_per = (long)p.NDT * NE, sv_step = (long)p.nwg * p.nsave * sv_per;  // save_index per value, step
  auto store_out = [&](int t, const float* src) {
    if (mode == 2) {  // [B,1,N,D]: the last step of the sequence only
      if (t0 + t == TT - 1 && el.real)
        st4s<OS>(a.states, last_index(p, el.b, tm.n, el.d), *reinterpret_cast<const f32x4*>(src + e0), of16);
      return;
    }
    // every staged value is read (unused ones too), so the reads form one burst
    f32x4 x[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) x[v] = *reinterpret_cast<const f32x4*>(src + v * NE + e0);
    if (!el.real) return;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (v >= S && !training) break;
      if (v < S && v >= nst) continue;  // the policy's states only: [nst,B,T,N,D]
      if (v < S) st4s<OS>(a.states, st_off[v] + t * st_step, x[v], of16);
      else st4s<SS>(a.save, sv_off + (v - S) * sv_per + t * sv_step, x[v], sf16);
    }
  };

  // Conversion of a landed raw slot into FP32 for the owners: lane l converts
  // four units of one row (the elements e0 .. e0+3 it also stores), one 8- or
  // 16-byte LDS read and one 16-byte write per gate. (The owners still add the
  // bias after Ry, in the reference's order: (x + Ry) + b and x + (b + Ry)
  // round differently, and a sLSTM max or clamp can break the other way.)
  auto convert = [&](int u) {
    const float* slot = xring + (long)(u % kFwdRing) * RING;
    float* dst = xf + (long)(u % kFwdXf) * Lds<CELL, NB>::XF;
    u32x4 raw[GW];
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      if constexpr (XS == 4) {
        raw[g] = *reinterpret_cast<const u32x4*>(slot + g * 256 + (lrow * 4 + lquad) * 4);
      } else {
        const uint2 h = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(slot + g * 256) +
                                                        (lrow * 4 + (lquad >> 1) * 2) * 16 + (lquad & 1) * 8);
        raw[g] = u32x4{h.x, h.y, 0u, 0u};
      }
    }
#pragma unroll
    for (int g = 0; g < GW; ++g) *reinterpret_cast<f32x4*>(dst + g * NE + e0) = cvt4s<XS>(raw[g], xf16);
  };
  // Per iteration t: barrier t; convert step t+2 (its loads went out in
  // iteration t-1; the owners read it after barrier t+1); issue the loads of
  // step t+P; drain step t-1. The loads go out right after the barrier: the
  // CU's vector memory returns data in issue order, so loads issued later would
  // hold up the compute waves' exchange polls behind them. VMEM operations
  // issued after the loads of step t+2 (t >= 2): the stores of iteration t-1.
  static_assert(P == 3, "the conversion waits assume the loads of step t+2 go out in iteration t-1");
  // stores per step: the policy's states (S, 1 or none in the loop) plus the saves when training
  constexpr int kStTrain = NV, kStTrainHidden = 1 + NSAVE, kStFull = S, kStHidden = 1;

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0, a.prof != nullptr);
  for (int u = 0; u < 2 && u < T; ++u) load_wx(u);
  wait_vm<0>();
  for (int u = 0; u < 2 && u < T; ++u) convert(u);
  lds_barrier();  // Wx of steps 0 and 1 converted; both raw slots read
  if (2 < T) load_wx(2);
  for (int t = 0; t < T; ++t) {
    prof.mark(0);
    prof.stamp(t, 0);
    lds_barrier();  // step t: outputs of step t-1 staged
    prof.mark(2);
    prof.stamp(t, 2);
    if (t + 2 < T) {
      if (t <= 1) wait_vm<0>();
      else {
        if (training && mode == 0) wait_vm<kStTrain>();
        else if (training) wait_vm<kStTrainHidden>();
        else if (mode == 0) wait_vm<kStFull>();
        else if (mode == 1) wait_vm<kStHidden>();
        else wait_vm<0>();
      }
      convert(t + 2);
    }
    prof.mark(1);
    prof.stamp(t, 1);
    // raw slot (t+3) % 2 held step t+1, converted before barrier t
    if (t + P < T) load_wx(t + P);
    if (t >= 1) store_out(t - 1, ost + ((t - 1) & 1) * NV * NE);
    prof.mark(3);
    prof.stamp(t, 3);
  }
  lds_barrier();  // outputs of the last step complete
  store_out(T - 1, ost + ((T - 1) & 1) * NV * NE);
  prof.acc[5] = T;
  prof.flush(a.prof);
  if (a.prof) prof.flush_trace(a.prof + 256, tm);
}

constexpr int kScoutLead = 6;  // step (iteration) a scout touches when step j is published: j + kScoutLead
constexpr uint32_t kScoutPatience = 1u << 12;  // polls a scout waits for one step
// Scout of a group, forward: touches the Wx lines of the group's real batch
// rows a few steps before the I/O waves load them (see bwd_scout), paced by
// the hidden-state word member 0 publishes each step.
template <int CELL, int MMA, bool PROJ>
__device__ void fwd_scout(const FwdArgs& a, const Team& tm, float* lds) {
  constexpr int GW = CellShape<CELL>::GW;
  const Plan& p = a.p;
  const int T = p.T, N = p.N, D = p.D, B = p.B;
  const int esz = p.dt_io == DT_F32 ? 4 : 2;
  const int b0 = tm.slab * p.BS, nreal = min(p.BS, B - b0);
  const int row_bytes = D * esz, lpr = (row_bytes + 127) / 128 + 1;  // lines of one row (+1: unaligned rows)
  const int nt = nreal * GW * lpr;
  auto lptr = (__attribute__((address_space(3))) void*)(lds + (threadIdx.x >> 6) * 64);
  auto touch = [&](int u) {
    const int nsc = p.nscout > 1 ? p.nscout : 1;
    for (int i = tm.member * blockDim.x + threadIdx.x; i < nt; i += nsc * blockDim.x) {
      const int r = i / (GW * lpr), g = (i / lpr) % GW, l = i % lpr;
      __builtin_amdgcn_global_load_lds(static_cast<const char*>(a.wx) + scout_wx_byte(p, tm.slab, tm.n, r, u, g, l, esz),
                                       lptr, 4, 0, 0);
    }
  };
  const char* xw = a.xbuf + (long)tm.group * p.BS * D * (MMA == MMA_F32 ? 8 : 4);
  const long xpar_b = (long)p.ngroups * p.BS * D * (MMA == MMA_F32 ? 8 : 4);
  auto published = [&](int t) {
    const uint32_t w = __hip_atomic_load(reinterpret_cast<const uint32_t*>(xw + (t & 1) * xpar_b) + (MMA == MMA_F32 ? 1 : 0),
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (MMA == MMA_F32 ? w : (w >> 16)) == step_tag(t);
  };
  // patience per step: a scout that loses the pace gives up within ~1 ms
  const uint32_t patience = a.spin_limit < kScoutPatience ? a.spin_limit : kScoutPatience;
  bool live = true;
  // projection-gated launches (plain loads only): touch step u only once its rows are complete
  int ready_rt = 0;
  auto ready = [&](int u) {
    if constexpr (PROJ) {
      const int need = proj_last_row_tile(u, B);
      uint32_t spins = 0;
      while (live && ready_rt <= need) {
        if (__hip_atomic_load(a.proj.ready + ready_rt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
            (uint32_t)a.proj.nct) {
          ++ready_rt;
          continue;
        }
        __builtin_amdgcn_s_sleep(2);
        if (++spins >= patience) live = false;
      }
    }
    return live;
  };
  for (int u = 3; u < kScoutLead && u < T; ++u)
    if (ready(u)) touch(u);
  for (int j = 0; live && j + kScoutLead < T; ++j) {
    uint32_t spins = 0;
    while (!published(j)) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins >= patience || ((spins & 255u) == 0 && load_status(a.status) != 0)) {
        live = false;
        break;
      }
    }
    if (live && ready(j + kScoutLead)) touch(j + kScoutLead);
  }
  __builtin_amdgcn_s_waitcnt(0);
}

template <int CELL, int MMA, int KTW, int NB, int NDT, int KSC, bool PROJ>
__global__ void __launch_bounds__(64 * (KSC + 1) * NDT) fwd_kernel(FwdArgs a) {
  using CS = CellShape<CELL>;
  constexpr int GR = CS::GR, GW = CS::GW, GT = CS::GT, S = CS::S;
  constexpr int NE = NB * 256, EPLMAX = (4 * NB + KSC - 1) / KSC, KS = KSC;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NV = Lds<CELL, NB>::NV, RING = Lds<CELL, NB>::RING;
  const Plan& p = a.p;
  extern __shared__ float lds[];
  Team tm;
  if constexpr (PROJ) {
    if (blockIdx.x >= p.grid) {  // beyond the recurrence's workgroups: input projection
      // workers on an XCD that hosts recurrence groups leave, so the groups keep
      // that XCD's L2 to themselves (the host clears every bit when no XCD is free)
      if (!((a.proj.skip_xcds >> (xcc_id() & 15u)) & 1u)) {
        if constexpr ((KSC + 1) * NDT >= 4) proj_wg_worker<MMA>(a.proj, reinterpret_cast<char*>(lds));
        else proj_wave_worker<MMA>(a.proj);
      }
      return;
    }
  }
  if (blockIdx.x >= p.grid - scout_blocks(p)) {  // a scout
    if (scout_setup(p, tm, a.claim, lds)) fwd_scout<CELL, MMA, PROJ>(a, tm, lds);
    return;
  }
  if (!team_setup(p, tm, a.claim, a.status, KSC, lds)) return;
  const int D = p.D, B = p.B, T = p.T, N = p.N;

  constexpr int RED_F = Lds<CELL, NB>::RED_F;
  float* red = lds + tm.team * Lds<CELL, NB>::fwd(KS);  // [2][KS][NB][272][4]
  float* xring = red + 2L * KS * NB * RED_F;            // [slot][gate][64][4]
  float* ost = xring + (long)kFwdRing * RING;           // [2][NV][NE]
  float* xf = ost + 2L * NV * NE;                       // [slot][gate][NE]

  // sLSTM: the reference's global predicate all(n0 == 0) over the call's whole initial state,
  // at the first step of a sequence only (a later window continues from a carry)
  uint32_t zflag = 0;
  if constexpr (CELL == CELL_SLSTM) {
    if (p.t0 == 0) {
      int nz = 0;
      const long cnt = (long)B * N * D;
      for (long i = threadIdx.x; i < cnt; i += blockDim.x) nz |= ld_val(a.s0, 2 * cnt + i, p.dt_state) != 0.f;
      zflag = __syncthreads_or(nz) ? 0u : 1u;
    }
  }
  if (tm.kw == KS) {
    // saved values: FP16 under the 16-bit policies (sLSTM: FP32), FP32 with FP32 operands
    constexpr int SS = SaveSize<CELL, MMA>::value;
    switch (io_sizes(p.dt_io, p.dt_out)) {
      case 0: fwd_io<CELL, MMA, NB, 2, 2, SS, PROJ>(a, tm, xring, ost, xf); break;
      case 1: fwd_io<CELL, MMA, NB, 2, 4, SS, PROJ>(a, tm, xring, ost, xf); break;
      default: fwd_io<CELL, MMA, NB, 4, 4, SS, PROJ>(a, tm, xring, ost, xf); break;
    }
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
  const int xgrp = tm.group * p.BS * D;  // this group's table
  const int cstride = 16 * p.BS;        // bytes between the chunks of a run
  int xword[NB][KTW];
  bool bval[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int bl = bt * 16 + tm.row;
    bval[bt] = tm.slab * p.BS + bl < B;
#pragma unroll
    for (int j = 0; j < KTW; ++j) xword[bt][j] = xgrp + xword_of<MMA>(p.BS, bl, (kt0 + j) * 32 + 8 * tm.kq);
  }
  const int xpar = p.ngroups * p.BS * D;  // words per parity
  // paired-poll runs (slab of <= 8 real rows, see gather_pair)
  const bool pair = NB == 1 && B <= 8;
  int xword_pair[KTW];
#pragma unroll
  for (int j = 0; j < KTW; ++j) xword_pair[j] = xgrp + xword_of<MMA>(p.BS, tm.lane & 7, (kt0 + j) * 32 + 8 * tm.kq);
  const bool bv_pair = (tm.lane & 7) < B;
  const int xkstride = xword_of<MMA>(p.BS, 0, 32) - xword_of<MMA>(p.BS, 0, 0);  // words between k-tiles

  // ---- owned elements
  int oe[EPLMAX];
  bool own[EPLMAX];
  Elem el[EPLMAX];
  float st[EPLMAX][S], bias[EPLMAX][GT];
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    own[s] = s * KS * 64 + tm.kw * 64 + tm.lane < NE;
    oe[s] = (NDT == 1 && CELL != CELL_SLSTM) ? owner_elem(s * KS * 64 + tm.kw * 64 + tm.lane)
                                             : s * KS * 64 + tm.kw * 64 + tm.lane;
    el[s] = elem_of(p, tm, oe[s] & (NE - 1));
    el[s].real = el[s].real && own[s];
#pragma unroll
    for (int k = 0; k < S; ++k)
      st[s][k] = el[s].real ? ld_val(a.s0, carry_index(p, k, el[s].b, tm.n, el[s].d), p.dt_state) : 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) bias[s][g] = own[s] ? ld_val(a.bias, ((long)g * N + tm.n) * D + el[s].d, p.dt_io) : 0.f;
  }

  // The initial hidden state goes through the exchange like any other step's:
  // step 0 polls the parity and tag of step -1.
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s)
    if (el[s].real) xstore<MMA>(xc, xpar + xgrp + xword_of<MMA>(p.BS, el[s].bl, el[s].d), st[s][0], step_tag(-1));

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0, a.prof != nullptr);
  // Retire every set-up load before the loop: the wait-count pass then sees no
  // load still pending at the loop head, and does not fence the exchange
  // stores inside the loop behind one.
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();  // Wx_0 in its slot
  // Wx of the next step, read from the ring right after each cell
  // Wx of the step, FP32, converted by the I/O wave (the reads are waited for
  // at the barrier, not here)
  float xnext[EPLMAX][GW];
  auto read_x = [&](int u) {
    const float* xr = xf + (long)(u % kFwdXf) * Lds<CELL, NB>::XF;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
#pragma unroll
      for (int g = 0; g < GW; ++g) xnext[s][g] = xr[g * NE + (oe[s] & (NE - 1))];
  };
  // The owners stage step t-1's outputs for the I/O wave and read step t's Wx
  // from the ring while step t's first poll is in flight (gather's `between`):
  // the poll goes out right after the loop head. The staging area of step t-1
  // is drained after barrier t, its ring slot was filled before barrier t-1.
  // Two-tile workgroups stage each step's outputs right after its cell instead
  // (slot t & 1, which the I/O wave drains after barrier t + 1) and read the
  // step's Wx with the partial sums: neither needs registers across the poll,
  // where these kernels run out
  constexpr bool kStageNow = NDT == 2;
  float sv_keep[EPLMAX][NSAVE];
  auto stage = [&](int t) {
    float* os = ost + (long)(t & 1) * NV * NE;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int e = oe[s];
#pragma unroll
      for (int k = 0; k < S; ++k) os[k * NE + e] = st[s][k];
#pragma unroll
      for (int v = 0; v < NSAVE; ++v) os[(S + v) * NE + e] = sv_keep[s][v];
    }
  };
  bool abort = false;
  for (int t = 0; t < T; ++t) {
    prof.stamp(t, 0);
    // ---- 1+2. h_{t-1} and the partial R . h over this wave's k-tiles
    f32x4 acc[NB][GR];
    auto zero = [&]() {
#pragma unroll
      for (int bt = 0; bt < NB; ++bt)
#pragma unroll
        for (int g = 0; g < GR; ++g) acc[bt][g] = f32x4{0.f, 0.f, 0.f, 0.f};
    };
    auto prod = [&](int bt, int j, const Frag<MMA>& f, int) {
#pragma unroll
      for (int g = 0; g < GR; ++g) acc[bt][g] = mma(A[g][j], f, acc[bt][g]);
    };
    auto between = [&]() {
      if (!kStageNow && t >= 1) stage(t - 1);
      if (!kStageNow) read_x(t);
    };
    {
      uint32_t polls;
      const int off = ((t - 1) & 1) * xpar;
      if (NB == 1 && pair) {
        // two-tile workgroups: the paired runs' words rebuilt each step from one
        // base (they are linear in the k-tile), so they hold no registers across
        // the loop where the unpaired runs are polled
        int xwp[KTW];
#pragma unroll
        for (int j = 0; j < KTW; ++j) xwp[j] = xword_pair[j];
        if constexpr (NDT == 2) {
          int bp = xword_pair[0];
          asm volatile("" : "+v"(bp));
#pragma unroll
          for (int j = 0; j < KTW; ++j) xwp[j] = bp + j * xkstride;
        }
        polls = gather_pair_mma<MMA, NDT, KTW>(xc, xwp, bv_pair, off, cstride, nkt, ptag(p, t - 1), a.status,
                                               a.spin_limit, abort, zero, prod, between);
      } else
        // pipelined chunks where the unpacked chunk fits beside the resident R
        // (GR * KTW <= 24: measured at D768 GRU 1.62 -> 1.58 ms; the LSTM's 32
        // spilled, 4.19 -> 4.92 ms)
        polls = gather_mma<MMA, NDT, NB, KTW, false, true, GR * KTW <= 24>(xc, xword, bval, off, cstride, nkt, ptag(p, t - 1), a.status,
                                              a.spin_limit, abort, zero, prod, between);
      prof.add(4, polls);
    }
    prof.mark(0);
    prof.stamp(t, 1);
    float* rp = red + (long)(t & 1) * KS * NB * RED_F;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < GR; ++g) v[g] = acc[bt][g][i];
        *reinterpret_cast<f32x4*>(rp + (tm.kw * NB + bt) * RED_F + red_slot(tm.lane * 4 + i) * 4) = v;
      }
    prof.mark(1);
    lds_barrier();
    prof.mark(2);
    prof.stamp(t, 2);

    // ---- 3. owners: gates, cell, exchange (the outputs are staged during the next poll)
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int e = oe[s];
      const int src = (e >> 8) * RED_F + red_slot(mfma_pos(e)) * 4;  // [bt][slot] -> 4 gates
      f32x4 part[KS];
#pragma unroll
      for (int w2 = 0; w2 < KS; ++w2) part[w2] = *reinterpret_cast<const f32x4*>(rp + w2 * NB * RED_F + src);
      float xcur[GW];
      if constexpr (kStageNow) {  // read with the partial sums (slot t % kFwdXf is kept until barrier t + 1)
        const float* xr = xf + (long)(t % kFwdXf) * Lds<CELL, NB>::XF;
#pragma unroll
        for (int g = 0; g < GW; ++g) xcur[g] = xr[g * NE + e];
      } else {
#pragma unroll
        for (int g = 0; g < GW; ++g) xcur[g] = xnext[s][g];
      }
      float ry[GR];
#pragma unroll
      for (int g = 0; g < GR; ++g) {
        float v = part[0][g];
#pragma unroll
        for (int w2 = 1; w2 < KS; ++w2) v += part[w2][g];
        ry[g] = v;
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
      // gradient_recurrent_clipval: the new hidden state is clamped (the saved
      // values are not: the backward passes straight through the clamp)
      if (p.flags & kFlagClip) st[s][0] = fminf(fmaxf(st[s][0], -p.clip), p.clip);
      // the exchange word goes out first: it is what the other workgroups wait for
      if (el[s].real && t + 1 < T)
        xstore<MMA>(xc, (t & 1) * xpar + xgrp + xword_of<MMA>(p.BS, el[s].bl, el[s].d), st[s][0], step_tag(t));
      if (s == 0) prof.stamp(t, 3);
#pragma unroll
      for (int v = 0; v < NSAVE; ++v) sv_keep[s][v] = sv[v];
      if constexpr (kStageNow) {
        float* os = ost + (long)(t & 1) * NV * NE;
#pragma unroll
        for (int k = 0; k < S; ++k) os[k * NE + e] = st[s][k];
#pragma unroll
        for (int v = 0; v < NSAVE; ++v) os[(S + v) * NE + e] = sv[v];
      }
    }
    prof.mark(3);
    prof.stamp(t, 4);
  }
  if (!kStageNow) stage(T - 1);
  lds_barrier();  // the I/O wave drains the last step

  // ---- carry: the last state in full precision
  if (a.carry) {
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
      if (el[s].real)
#pragma unroll
        for (int k = 0; k < S; ++k)
          st_val(a.carry, carry_index(p, k, el[s].b, tm.n, el[s].d), p.dt_state, st[s][k]);
  }
  prof.acc[5] = T;
  prof.flush(a.prof);
  if (a.prof) prof.flush_trace(a.prof + 256, tm);
}

// ===================================================================== backward
// I/O wave of a team. Per iteration it (step t = T-1-it), before barrier it:
// stage the inputs of iteration it+2 (state cotangents and saved values,
// converted to FP32) from registers into LDS slot (it+2) % 3, then issue the
// loads of iteration it+4 into the registers just freed; after barrier it:
// drain iteration it's outputs (dWx, GRU: candidate cotangents). Every LDS
// access is lane-contiguous (value-major layouts). XS, OS, SS: element sizes
// (2 or 4 bytes) of dWx, of the state cotangents and of the saved values,
// fixed at compile time (see fwd_io).
template <int CELL, int MMA, int NB, int XS, int OS, int SS>
__device__ void bwd_io(const BwdArgs& a, const Team& tm, float* iring, float* ost) {
  static_assert(NB == 1, "one 16-row batch tile per group");
  using CS = CellShape<CELL>;
  constexpr int GW = CS::GW, S = CS::S, NE = NB * 256, PR = kBwdRegs;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NIN = S + NSAVE, NOB = Lds<CELL, NB>::NOB;
  const Plan& p = a.p;
  const int T = p.T, N = p.N, D = p.D, B = p.B;
  const bool xf16 = p.dt_io == DT_F16, of16 = p.dt_out == DT_F16, sf16 = p.dt_save == DT_F16;
  const bool hidden_only = (p.flags & kFlagOutHidden) != 0;  // d_states [B,T,N,D]: the hidden state's only
  const int e0 = io_elem(tm.lane, 0);
  const Elem el = elem_of(p, tm, e0);
  // per-lane element offsets at step 0, and their step strides
  const long ds_off = (((long)el.b * T) * N + tm.n) * D + el.d;  // + k * B*T*N*D + t * N*D
  const long ds_k = (long)B * T * N * D, ds_t = (long)N * D;
  const long sv_off = save_index(p, NE, 0, tm.wgi, 0, tm.team, e0);
  const long sv_v = (long)p.NDT * NE, sv_t = (long)p.nwg * p.nsave * sv_v;
  const long wx_off = ((long)el.b * T) * GW * N * D + (long)tm.n * D + el.d;  // + t * GW*N*D + g * N*D
  const long wx_t = (long)GW * N * D, wx_g = (long)N * D;
  const bool has_ds = a.d_states != nullptr;
  auto load_in = [&](int it, u32x4 (&dst)[NIN]) {
    const long t = T - 1 - it;
#pragma unroll
    for (int k = 0; k < S; ++k)
      dst[k] = (el.real && has_ds && (k == 0 || !hidden_only)) ? ld4s<OS>(a.d_states, ds_off + k * ds_k + t * ds_t)
                                                               : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int v = 0; v < NSAVE; ++v)
      dst[S + v] = el.real  // padding rows were not saved
                       ? ld4s<SS>(a.save, sv_off + v * sv_v + t * sv_t)
                       : u32x4{0u, 0u, 0u, 0u};
  };
  auto stage = [&](int it, const u32x4 (&src)[NIN]) {
    float* slot = iring + (long)(it % kBwdStage) * NIN * NE;
#pragma unroll
    for (int k = 0; k < NIN; ++k)
      *reinterpret_cast<f32x4*>(slot + k * NE + e0) = k < S ? cvt4s<OS>(src[k], of16) : cvt4s<SS>(src[k], sf16);
  };
  auto store_out = [&](int it, const float* src) {
    const long t = T - 1 - it;
    f32x4 o[NOB];
#pragma unroll
    for (int g = 0; g < NOB; ++g) o[g] = *reinterpret_cast<const f32x4*>(src + g * NE + e0);
    if (!el.real) return;
#pragma unroll
    for (int g = 0; g < GW; ++g) st4s<XS>(a.dwx, wx_off + t * wx_t + g * wx_g, o[g], xf16);
    if constexpr (CELL == CELL_GRU)  // the R-only candidate gate's cotangent, for the dR GEMM
      *reinterpret_cast<f32x4*>(a.dcand + ((long)el.b * T + t) * N * D + (long)tm.n * D + el.d) = o[3];
  };

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0, a.prof != nullptr);
  u32x4 buf[PR][NIN];  // indexed with constants only (unrolled loops), so it stays in registers
#pragma unroll
  for (int j = 0; j < PR; ++j)
    if (j < T) load_in(j, buf[j]);
#pragma unroll
  for (int j = 0; j < PR; ++j) {
    if (j < T) stage(j, buf[j]);
    if (j + PR < T) load_in(j + PR, buf[j]);
  }
  lds_barrier();  // inputs of iterations 0 and 1 staged
  for (int it0 = 0; it0 < T; it0 += PR) {
#pragma unroll
    for (int j = 0; j < PR; ++j) {
      const int it = it0 + j;
      if (it < T) {
        if (it + PR < T) {
          stage(it + PR, buf[j]);  // buf[j] holds iteration it + 2 (loaded two iterations ago)
          prof.mark(0);
          prof.stamp(it, 0);
          if (it + 2 * PR < T) load_in(it + 2 * PR, buf[j]);
          prof.mark(1);
          prof.stamp(it, 1);
        }
        lds_barrier();  // iteration it: outputs staged; inputs of it+2 staged
        prof.mark(2);
        prof.stamp(it, 2);
        store_out(it, ost + (long)(it & 1) * NOB * NE);
        prof.mark(3);
        prof.stamp(it, 3);
      }
    }
  }
  prof.acc[5] = T;
  prof.flush(a.prof ? a.prof + 128 : nullptr);
  if (a.prof) prof.flush_trace(a.prof + 256 + 128 * 16 * 64, tm);
}

// Scout of a group (backward; one extra workgroup on the group's XCD): it
// touches the lines the group's I/O waves will load a few iterations later
// (state cotangents of the real batch rows, saved values), so those loads hit
// the XCD's L2 instead of HBM. A CU's vector memory returns data in issue
// order, so an HBM load in an I/O wave holds up every exchange poll of its CU
// issued after it; the scout, on a CU of its own, takes that latency instead.
// The touches are LDS-DMA loads (no registers in flight; the LDS content is
// never read). The scout paces itself by the exchange word that member 0
// publishes each iteration; nothing waits for it, and every wait of its own is
// bounded (spin limit, sticky status), so it always finishes.
// RS: the reduce-scatter backward (frnn_bwd_rs.h), whose exchange table holds
// 32-bit split words of partial sums, [v][p][b][w] per group.
template <int CELL, int MMA, bool RS = false>
__device__ void bwd_scout(const BwdArgs& a, const Team& tm, float* lds) {
  using CS = CellShape<CELL>;
  constexpr int S = CS::S, GR = CS::GR;
  const Plan& p = a.p;
  const int T = p.T, N = p.N, D = p.D, B = p.B, NE = p.NB * 256;
  const int nst = a.d_states ? ((p.flags & kFlagOutHidden) ? 1 : S) : 0;
  const int esz = p.dt_out == DT_F32 ? 4 : 2;
  const int b0 = tm.slab * p.BS, nreal = min(p.BS, B - b0);
  const int row_bytes = D * esz, lpr = (row_bytes + 127) / 128 + 1;  // lines of one row (+1: unaligned rows)
  const int nd = nst * nreal * lpr;                                    // state-cotangent touches
  const int ssz = p.dt_save == DT_F32 ? 4 : 2;                         // bytes of a saved value
  const int lpt = 2 * ssz;                                             // lines of a 16-row tile of one value
  const int nall = bwd_scout_lines(p, nst, nreal, esz, ssz);           // nd + the save touches
  const int nsc = p.nscout > 1 ? p.nscout : 1;
  auto lptr = (__attribute__((address_space(3))) void*)(lds + (threadIdx.x >> 6) * 64);
  auto touch = [&](int it) {
    const int t = T - 1 - it;
    for (int i = tm.member * blockDim.x + threadIdx.x; i < nall; i += nsc * blockDim.x) {
      const char* src = nullptr;
      if (i < nd) {
        const int k = i / (nreal * lpr), r = (i / lpr) % nreal, l = i % lpr;
        const long e0 = ((((long)k * B + b0 + r) * T + t) * N + tm.n) * D;
        src = static_cast<const char*>(a.d_states) + e0 * esz + min(128 * l, row_bytes - 4);
      } else {
        const int j = i - nd, l = j % lpt, bt = (j / lpt) % p.NB, rest = (j / lpt) / p.NB;
        const int team = rest % p.NDT, v = (rest / p.NDT) % p.nsave, m = rest / (p.NDT * p.nsave);
        const int rows = min(max(nreal - bt * 16, 0), 16);  // real rows of this 16-row tile
        if (l * (8 / ssz) < rows)  // a 128-byte line holds 8 / ssz rows of 16 units
          src = static_cast<const char*>(a.save) +
                save_index(p, NE, t, tm.group * p.wpg + m, v, team, bt * 256) * ssz + 128 * l;
      }
      if (src) __builtin_amdgcn_global_load_lds(src, lptr, 4, 0, 0);
    }
  };
  // the word of (row 0, k 0) of the group's table (RS: of p 0, row 0, producer 0), parity by parity
  const long tbl = RS ? (long)D * 16 * p.wpg * 4 : (long)p.BS * GR * D * (MMA == MMA_F32 ? 8 : 4);
  const char* xw = a.xbuf + (long)tm.group * tbl;
  const long xpar_b = (long)p.ngroups * tbl;
  auto published = [&](int it) {
    const char* w = xw + (it & 1) * xpar_b;
    uint32_t tag;
    if constexpr (MMA == MMA_F32 && !RS) tag = __hip_atomic_load(reinterpret_cast<const uint32_t*>(w) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else tag = __hip_atomic_load(reinterpret_cast<const uint32_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 3u;
    return tag == step_tag(it);
  };
  // Every wave paces itself (a barrier-paced variant measured slower).
  for (int x = 3; x < kScoutLead && x < T; ++x) touch(x);
  // patience per step: a scout that loses the pace gives up within ~1 ms
  const uint32_t patience = a.spin_limit < kScoutPatience ? a.spin_limit : kScoutPatience;
  bool live = true;
  for (int j = 0; live && j + kScoutLead < T; ++j) {
    uint32_t spins = 0;
    while (!published(j)) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins >= patience || ((spins & 255u) == 0 && load_status(a.status) != 0)) {
        live = false;
        break;
      }
    }
    if (live) touch(j + kScoutLead);
  }
  __builtin_amdgcn_s_waitcnt(0);
}

template <int CELL, int MMA, int KTW, int NB, int NDT, int KSC>
__global__ void __launch_bounds__(64 * (KSC + 1) * NDT) bwd_kernel(BwdArgs a) {
  using CS = CellShape<CELL>;
  constexpr int GR = CS::GR, GW = CS::GW, GT = CS::GT, S = CS::S;
  constexpr int NE = NB * 256, EPLMAX = (4 * NB + KSC - 1) / KSC, KS = KSC;
  constexpr int NSAVE = Cell<CELL>::NSAVE, NIN = S + NSAVE;
  constexpr int NOB = Lds<CELL, NB>::NOB;
  constexpr int NF = GR * KTW;  // max fragments of R^T per wave
  const Plan& p = a.p;
  extern __shared__ float lds[];
  Team tm;
  if (blockIdx.x >= p.grid - scout_blocks(p)) {  // a scout
    if (scout_setup(p, tm, a.claim, lds)) bwd_scout<CELL, MMA>(a, tm, lds);
    return;
  }
  if (!team_setup(p, tm, a.claim, a.status, KSC, lds)) return;
  const int D = p.D, B = p.B, N = p.N, T = p.T;
  const int GD = GR * D;
  const bool cut = (p.flags & kFlagCut) != 0;
  const bool v1 = CELL == CELL_SLSTM && (p.flags & kFlagV1Grad) != 0;
  // 16-bit paths: the gate cotangents travel as split words (hi + lo operands),
  // so R^T dG is not computed from rounded dG (the reference's policy rounds the
  // hidden state's cotangent after the product, not dG before it). Measured at
  // C2: +0.17 ms of backward over BF16 words.
  constexpr bool kSplit = MMA != MMA_F32;
  // Polls check their tags before they unpack and multiply: a stale poll (the
  // backward averages up to 2 per step) repeats at once instead of after a
  // wasted product. Measured at C2: -0.17 ms against speculative products.
  constexpr bool kSpecB = false;

  constexpr int RED_B = Lds<CELL, NB>::RED_B;
  float* red = lds + tm.team * Lds<CELL, NB>::bwd(KS);  // [2][NB][KS][304]
  float* iring = red + 2L * NB * KS * RED_B;             // [3][NIN][NE]
  float* ost = iring + (long)kBwdStage * NIN * NE;       // [2][NOB][NE]
  // [owner wave]: last step it published (an LDS pointer: generic atomics would be flat operations)
  __attribute__((address_space(3))) uint32_t* pubf =
      (__attribute__((address_space(3))) uint32_t*)reinterpret_cast<uint32_t*>(ost + 2L * NOB * NE);

  if (tm.kw == KS) {
    // saved values: FP16 under the 16-bit policies (sLSTM: FP32), FP32 with FP32 operands
    constexpr int SS = SaveSize<CELL, MMA>::value;
    switch (io_sizes(p.dt_io, p.dt_out)) {
      case 0: bwd_io<CELL, MMA, NB, 2, 2, SS>(a, tm, iring, ost); break;
      case 1: bwd_io<CELL, MMA, NB, 2, 4, SS>(a, tm, iring, ost); break;
      default: bwd_io<CELL, MMA, NB, 4, 4, SS>(a, tm, iring, ost); break;
    }
    return;
  }

  Xchg xc;
  {
    // Held in VGPRs (backward only: measured slower in the forward): under
    // SGPR pressure the compiler otherwise reloads the pointer from the kernel
    // arguments inside the time loop, and the scalar load's wait lands in
    // front of the exchange stores.
    uintptr_t xb = reinterpret_cast<uintptr_t>(a.xbuf);
    asm("" : "+v"(xb));
    xc.base = reinterpret_cast<char*>(xb);
  }
  xc.shared_xcd = (p.flags & 2) ? 1 : 0;
  xc.rsrc = __builtin_amdgcn_make_buffer_rsrc(a.xbuf, 0, (int)a.xbytes, 0x00020000);

  // ---- contraction split over the (g, o) k-tiles of dG: [kt0, kt0 + nkt) of GR*D/32
  const int KT = p.kt_bwd;
  const int kt0 = (tm.kw * KT) / KS;
  const int nkt = ((tm.kw + 1) * KT) / KS - kt0;
  // A wave without k-tiles (G_R*D/32 < KS: only the GRU, at D = 32, three
  // k-tiles over four waves; the Elman's NF == 1 gather handles it) skips the
  // gather, whose NF > 1 paths would also skip the prefetch of its next inputs;
  // it adds a zero partial. (nkt is the same in every lane; read from the first
  // lane, the branch stays a scalar one. The other cells keep the plain cut
  // test: the extra condition measured 3% slower in the LSTM backward.)
  const bool nopoll = cut || (CELL == CELL_GRU && __builtin_amdgcn_readfirstlane(nkt) <= 0);

  // ---- resident R^T: A[j][row = p][k = (o, g)] = R[g, n, o, dt*16 + row]
  Frag<MMA> A[NF];
#pragma unroll
  for (int j = 0; j < NF; ++j) {
    A[j].zero();
    if (j < nkt) {
      const int kk = (kt0 + j) * 32 + 8 * tm.kq;  // k = o * GR + g: an element's gates are adjacent
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int g = (kk + i) % GR, o = (kk + i) / GR;
        frag_set(A[j], i, ld_val(a.R, (((long)g * N + tm.n) * D + o) * D + tm.dt * 16 + tm.row, p.dt_io));
      }
    }
  }

  const int xgrp = tm.group * p.BS * GD;  // this group's table
  const int cstride = 16 * p.BS;         // bytes between the chunks of a run
  int xword[NB][NF];
  bool bval[NB];
#pragma unroll
  for (int bt = 0; bt < NB; ++bt) {
    const int bl = bt * 16 + tm.row;
    bval[bt] = tm.slab * p.BS + bl < B;
#pragma unroll
    for (int j = 0; j < NF; ++j) xword[bt][j] = xgrp + xword_of<MMA>(p.BS, bl, (kt0 + j) * 32 + 8 * tm.kq);
  }
  const int xpar = p.ngroups * p.BS * GD;
  const bool pair = NB == 1 && B <= 8;
  int xword_pair[NF];
#pragma unroll
  for (int j = 0; j < NF; ++j) xword_pair[j] = xgrp + xword_of<MMA>(p.BS, tm.lane & 7, (kt0 + j) * 32 + 8 * tm.kq);
  const bool bv_pair = (tm.lane & 7) < B;

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
                        ? ld_val(a.d_carry, carry_index(p, k, el[s].b, tm.n, el[s].d), p.dt_state)
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

  Prof prof;
  prof.init(a.prof != nullptr && blockIdx.x == 0, a.prof != nullptr);
  // Waves that own no element (KS > 4) start their poll late: polled at the
  // loop head, the exchange is stale, and the re-polls hold the CU's in-order
  // memory returns and the SIMDs the owners' pointwise runs on. Measured (LSTM
  // backward): with at most 8 batch rows (paired polls) a fixed delay is best
  // (C2 1.61 -> 1.52 ms; waiting for the owners' flag in LDS 1.58 ms). With the
  // paired reduction reads, s_sleep 11 (~700 cycles) is best at C2: 1.525 ms
  // at 8, 1.50 at 10, 1.487 at 11, 1.50 at 12, 1.54 at 13, 1.58 at 6 and at 16.
  // With 16 rows, waiting for the owners' flag is best (B16 N2 D384 3.81 ->
  // 3.43 ms, N1 D512 4.53 -> 4.22 ms; the fixed delay 3.59 and 4.28 ms),
  // checked every ~130 cycles (s_sleep 2; against 4, B16 T1024 backward over
  // two runs: D128 N6 1.78 -> 1.72 ms, D256 N3 2.26 -> 2.15-2.21, D384 N2 3.33
  // -> 3.24-3.29, D512 N1 4.37 -> 4.29-4.33).
  constexpr int kOwnerWaves = (NE + 63) / 64 < KS ? (NE + 63) / 64 : KS;
  if (tm.kw == 0 && tm.lane < kOwnerWaves) pubf[tm.lane] = 0u;
  __builtin_amdgcn_s_waitcnt(0);  // no set-up load pending at the loop head (see the forward kernel)
  lds_barrier();  // inputs of iterations 0 and 1 staged by the I/O wave; the flags clear
  // One-tile workgroups read the owners' inputs of the next iteration from LDS
  // during this iteration's poll (the I/O wave staged them before the previous
  // barrier), so no LDS read stands between the loop head and the pointwise
  // backward. Two-tile workgroups (two elements per lane, 256 registers a wave)
  // have no registers for a second set and read them at the loop head, and so
  // does the LSTM with two or more k-tiles per wave in eight waves (168
  // registers a wave): the second set made it spill, B16 T1024 backward D512
  // 4.19 -> 3.83 ms and N2 D384 3.45 -> 2.98 ms without it (the GRU and sLSTM
  // there were 5-9% slower without it).
  constexpr bool kPrefetch = NDT == 1 && !(CELL == CELL_LSTM && KS == 8 && KTW >= 2);
  float in_cur[EPLMAX][NIN], in_next[kPrefetch ? EPLMAX : 1][NIN];
  auto read_in = [&](int it, auto& dst) {
    const float* ir = iring + (long)(it % kBwdStage) * NIN * NE;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s)
#pragma unroll
      for (int k = 0; k < NIN; ++k) dst[s][k] = own[s] ? ir[k * NE + oe[s]] : 0.f;
  };
  read_in(0, in_cur);
  // sLSTM: (c_{t-1}, n_{t-1}) of iteration j are c and n of step t-1, saved in
  // the inputs of iteration j+1 (the initial state at the last iteration); they
  // are read during the previous iteration's reduction, once the barrier has
  // made that ring slot complete
  float prev_cn[EPLMAX][2];
  auto read_prev = [&](int j) {
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      const float* irn = iring + (long)((j + 1) % kBwdStage) * NIN * NE;
#pragma unroll
      for (int k = 0; k < 2; ++k)
        prev_cn[s][k] = CELL != CELL_SLSTM ? 0.f : (j + 1 < T ? (own[s] ? irn[(S + 1 + k) * NE + oe[s]] : 0.f)
                                                              : init_cn[s][k]);
    }
  };
  read_prev(0);
  bool abort = false;
  for (int it = 0; it < T; ++it) {
    prof.stamp(it, 0);
    const int xoff = (it & 1) * xpar;
    if constexpr (!kPrefetch)
      if (it > 0) read_in(it, in_cur);
    // ---- 1. owners: pointwise backward of step t = T-1-it, publish dG_t
    float* os = ost + (long)(it & 1) * NE * NOB;
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int e = oe[s];
      const float* in = in_cur[s];
      float ds[S];
#pragma unroll
      for (int k = 0; k < S; ++k) ds[k] = carry[s][k] + in[k];
      if (p.flags & kFlagClip) {
        // the recurrent cotangent of h_t (direct path + R^T dG of step t+1) is
        // clamped before the caller's cotangent is added; at the first
        // iteration carry[0] is the caller's cotangent of the last state
        const float rec = carry[s][0] + dhrec[s];
        ds[0] = (it == 0 ? rec : fminf(fmaxf(rec, -p.clip), p.clip)) + in[0];
      } else {
        ds[0] += dhrec[s];
      }
      float sv[NSAVE];
#pragma unroll
      for (int v = 0; v < NSAVE; ++v) sv[v] = in[S + v];
      float dry[GR], dwx[GW], db[GT], cr[S];
      Cell<CELL>::bwd(ds, sv, prev_cn[s], dry, dwx, db, cr, v1);
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
      // the element's gate cotangents go out first (k = o * GR + g: one vector store when GR = 4)
      if (el[s].real && !cut) {
        if constexpr (MMA != MMA_F32 && GR == 4) {  // k = 4d .. 4d+3: one aligned chunk
          xstore_vec<MMA, GR, kSplit>(xc, xoff + xgrp + xword_of<MMA>(p.BS, el[s].bl, el[s].d * GR), dry,
                                      step_tag(it));
        } else {
#pragma unroll
          for (int g = 0; g < GR; ++g)
            xstore<MMA, kSplit>(xc, xoff + xgrp + xword_of<MMA>(p.BS, el[s].bl, el[s].d * GR + g), dry[g],
                                step_tag(it));
        }
      }
      // then the outputs the I/O wave drains after the barrier (value-major)
#pragma unroll
      for (int g = 0; g < GW; ++g) os[g * NE + e] = dwx[g];
      if constexpr (CELL == CELL_GRU) os[3 * NE + e] = dry[0];
    }
    if constexpr (KS > kOwnerWaves)
      if (!pair && tm.kw < kOwnerWaves && tm.lane == 0)  // (the paired polls wait a fixed delay instead)
        __hip_atomic_store(pubf + tm.kw, (uint32_t)it + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    prof.mark(3);
    prof.stamp(it, 1);

    // ---- 2. dh_{t-1} partial = R^T dG_t over this wave's k-tiles, fused with the poll
    f32x4 acc[NB];
    auto zero = [&]() {
#pragma unroll
      for (int bt = 0; bt < NB; ++bt) acc[bt] = f32x4{0.f, 0.f, 0.f, 0.f};
    };
    // split words: the hi and lo products go into one accumulator (a second
    // accumulator for the lo products measured slower)
    auto prod = [&](int bt, int j, const Frag<MMA>& f, int) { acc[bt] = mma(A[j], f, acc[bt]); };
    uint32_t polls = 0;
    // the next iteration's inputs, read while the first poll is in flight
    auto between = [&]() {
      if constexpr (kPrefetch)
        if (it + 1 < T) read_in(it + 1, in_next);
    };
    if constexpr (KS > kOwnerWaves) {
      if (tm.kw >= kOwnerWaves && !cut) {
        if (pair) {
          __builtin_amdgcn_s_sleep(11);
        } else {
          // bounded: the owners raise their flags every iteration
          for (uint32_t w = 0; w < (1u << 20); ++w) {
            bool pub = true;
#pragma unroll
            for (int k = 0; k < kOwnerWaves; ++k)
              pub &= __hip_atomic_load(pubf + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) > (uint32_t)it;
            if (pub) break;
            __builtin_amdgcn_s_sleep(2);
          }
        }
      }
    }
    if (nopoll) {  // gradient_recurrent_cut (no R^T dG reaches h_{t-1}), or no k-tiles
      zero();
      between();
    } else if (NB == 1 && pair) {
      polls = gather_pair_mma<MMA, NDT, NF, kSplit, kSpecB>(xc, xword_pair, bv_pair, xoff, cstride, nkt, ptag(p, it),
                                                            a.status, a.spin_limit, abort, zero, prod, between);
    } else {
      polls = gather_mma<MMA, NDT, NB, NF, kSplit, kSpecB>(xc, xword, bval, xoff, cstride, nkt, ptag(p, it),
                                                           a.status, a.spin_limit, abort, zero, prod, between);
    }
    // paired split-word products: columns 8-15 hold the lo products of rows 0-7
    if constexpr (kSplit && NB == 1)
      if (pair && !nopoll) acc[0] = fold_cols8(acc[0]);
    prof.add(4, polls);
    prof.mark(0);
    prof.stamp(it, 2);
    float* rp = red + (long)(it & 1) * NB * KS * RED_B;
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
      *reinterpret_cast<f32x4*>(rp + (bt * KS + tm.kw) * RED_B + red_idx(tm.lane * 4)) = acc[bt];
    prof.mark(1);
    lds_barrier();
    prof.mark(2);
    prof.stamp(it, 3);

    // ---- 3. owners: reduce -> recurrent cotangent of h_{t-1}
    if constexpr (CELL == CELL_SLSTM)
      if (it + 1 < T) read_prev(it + 1);  // its ring slot was staged before this barrier
#pragma unroll
    for (int s = 0; s < EPLMAX; ++s) {
      if (!own[s]) continue;
      const int src = (oe[s] >> 8) * KS * RED_B + red_idx(mfma_pos(oe[s]));
      float part[KS];
#pragma unroll
      for (int w2 = 0; w2 < KS; ++w2) part[w2] = rp[src + w2 * RED_B];
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < KS; ++w2) v += part[w2];
      // the BF16 policy rounds the cotangent of the rounded hidden operand
      dhrec[s] = el[s].real ? round_op<MMA>(v) : 0.f;
    }
    if constexpr (kPrefetch) {
#pragma unroll
      for (int s = 0; s < EPLMAX; ++s)
#pragma unroll
        for (int k = 0; k < NIN; ++k) in_cur[s][k] = in_next[s][k];
    }
    prof.mark(6);
    prof.stamp(it, 4);
  }

  // ---- d(initial state), d(bias) partials
#pragma unroll
  for (int s = 0; s < EPLMAX; ++s) {
    if (!own[s]) continue;
    if (el[s].real) {
#pragma unroll
      for (int k = 0; k < S; ++k)
        st_val(a.ds0, carry_index(p, k, el[s].b, tm.n, el[s].d), p.dt_state,
               carry[s][k] + (k == 0 ? dhrec[s] : 0.f));
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

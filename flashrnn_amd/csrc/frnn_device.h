// Device-side building blocks of the gfx950 fused recurrence.
//
// Execution model (see frnn_plan.h for the host side of the same plan):
//  * a "group" is one head n and one batch slab of 16*NB rows; it owns the
//    whole recurrence of that slab and never talks to another group;
//  * a group is D/16 workgroups, one per 16-wide tile of hidden units; all of
//    them run on one XCD (workgroup w runs on XCD w % 8), so they share an L2;
//  * inside a workgroup, KS waves split the contraction (K) dimension of the
//    per-step product and reduce their partial sums through LDS;
//  * each step, every workgroup publishes its slice of the new hidden state
//    (forward) or of the gate cotangent dG (backward) into an exchange buffer
//    in L2 as tagged words; readers poll those words until the tag of the
//    step arrives. That is the whole grid "barrier": no counters, no flags.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "frnn_plan.h"

namespace frnn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

enum { CELL_LSTM = 0, CELL_GRU = 1, CELL_ELMAN = 2, CELL_SLSTM = 3 };
// Recurrent-product operand types; MMA_BF16 and MMA_F16 are the 16-bit family
// (same exchange words and layouts, their own conversions and MFMA).
enum { MMA_BF16 = 0, MMA_F32 = 1, MMA_F16 = 2 };
enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
enum { ST_OK = 0, ST_TIMEOUT = 5, ST_PLACEMENT = 6 };

// Cell shapes: recurrent gates, input gates, bias gates, states.
template <int CELL> struct CellShape;
template <> struct CellShape<CELL_LSTM> { static constexpr int GR = 4, GW = 4, GT = 4, S = 2; };
template <> struct CellShape<CELL_GRU> { static constexpr int GR = 3, GW = 3, GT = 4, S = 1; };
template <> struct CellShape<CELL_ELMAN> { static constexpr int GR = 1, GW = 1, GT = 1, S = 1; };
template <> struct CellShape<CELL_SLSTM> { static constexpr int GR = 4, GW = 4, GT = 4, S = 4; };

// ------------------------------------------------------------------ numbers
__device__ __forceinline__ uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float u2f(uint32_t x) { return __builtin_bit_cast(float, x); }

// FP32 -> BF16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ uint32_t bf16_bits(float x) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)x);
}
__device__ __forceinline__ float bf16_to_f32(uint32_t bits) { return u2f(bits << 16); }
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(bf16_bits(x)); }
// FP32 -> FP16 bits, round to nearest even (v_cvt_f16_f32), and back.
__device__ __forceinline__ uint32_t f16_bits(float x) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)x);
}
__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
}
__device__ __forceinline__ float round_f16(float x) { return f16_to_f32(f16_bits(x)); }
// A 16-bit value of dtype dt (DT_BF16 or DT_F16) <-> FP32.
__device__ __forceinline__ uint32_t h16_bits(float x, int dt) { return dt == DT_F16 ? f16_bits(x) : bf16_bits(x); }
__device__ __forceinline__ float h16_to_f32(uint32_t bits, int dt) {
  return dt == DT_F16 ? f16_to_f32(bits & 0xffffu) : bf16_to_f32(bits & 0xffffu);
}

// Loads/stores of the public tensors in their runtime dtype.
__device__ __forceinline__ float ld_val(const void* p, long i, int dt) {
  if (dt == DT_F32) return static_cast<const float*>(p)[i];
  return h16_to_f32(static_cast<const unsigned short*>(p)[i], dt);
}
__device__ __forceinline__ void st_val(void* p, long i, int dt, float v) {
  if (dt == DT_F32) static_cast<float*>(p)[i] = v;
  else static_cast<unsigned short*>(p)[i] = (unsigned short)h16_bits(v, dt);
}

// Four consecutive values, raw: loads issue now and convert later (raw4_f32),
// so an in-flight load is not waited for at its issue point.
__device__ __forceinline__ u32x4 ld4_raw(const void* p, long i, int dt) {
  if (dt == DT_F32) return *reinterpret_cast<const u32x4*>(static_cast<const float*>(p) + i);
  const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const unsigned short*>(p) + i);
  return u32x4{u.x, u.y, 0u, 0u};
}
__device__ __forceinline__ f32x4 raw4_f32(u32x4 r, int dt) {
  if (dt == DT_F32) return f32x4{u2f(r[0]), u2f(r[1]), u2f(r[2]), u2f(r[3])};
  if (dt == DT_F16)
    return f32x4{f16_to_f32(r[0] & 0xffffu), f16_to_f32(r[0] >> 16), f16_to_f32(r[1] & 0xffffu),
                 f16_to_f32(r[1] >> 16)};
  return f32x4{u2f(r[0] << 16), u2f(r[0] & 0xffff0000u), u2f(r[1] << 16), u2f(r[1] & 0xffff0000u)};
}

// Four consecutive values (16-byte aligned in FP32, 8-byte aligned in 16 bits).
__device__ __forceinline__ f32x4 ld4(const void* p, long i, int dt) {
  if (dt == DT_F32) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const unsigned short*>(p) + i);
  return raw4_f32(u32x4{u.x, u.y, 0u, 0u}, dt);
}
__device__ __forceinline__ void st4(void* p, long i, int dt, f32x4 v) {
  if (dt == DT_F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = v;
  } else {
    uint2 u;
    u.x = h16_bits(v[0], dt) | (h16_bits(v[1], dt) << 16);
    u.y = h16_bits(v[2], dt) | (h16_bits(v[3], dt) << 16);
    *reinterpret_cast<uint2*>(static_cast<unsigned short*>(p) + i) = u;
  }
}

// Four consecutive values of SZ bytes each, with the element size fixed at
// compile time (SZ = 4: FP32; SZ = 2: BF16, or FP16 when f16): loads move raw
// bits and conversions are branch-free selects, so no load waits at a dtype
// branch (a value merged from two branches is "used" at the merge, which
// makes the compiler wait for the load there).
template <int SZ>
__device__ __forceinline__ u32x4 ld4s(const void* p, long i) {
  if constexpr (SZ == 4) {
    return *reinterpret_cast<const u32x4*>(static_cast<const float*>(p) + i);
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const unsigned short*>(p) + i);
    return u32x4{u.x, u.y, 0u, 0u};
  }
}
template <int SZ>
__device__ __forceinline__ f32x4 cvt4s(u32x4 r, bool f16) {
  if constexpr (SZ == 4) {
    return __builtin_bit_cast(f32x4, r);
  } else {
    const f32x4 b = {u2f(r[0] << 16), u2f(r[0] & 0xffff0000u), u2f(r[1] << 16), u2f(r[1] & 0xffff0000u)};
    const f32x4 h = {f16_to_f32(r[0] & 0xffffu), f16_to_f32(r[0] >> 16), f16_to_f32(r[1] & 0xffffu),
                     f16_to_f32(r[1] >> 16)};
    return f16 ? h : b;
  }
}
template <int SZ>
__device__ __forceinline__ void st4s(void* p, long i, f32x4 v, bool f16) {
  if constexpr (SZ == 4) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = v;
  } else {
    const uint2 b = {bf16_bits(v[0]) | (bf16_bits(v[1]) << 16), bf16_bits(v[2]) | (bf16_bits(v[3]) << 16)};
    const uint2 h = {f16_bits(v[0]) | (f16_bits(v[1]) << 16), f16_bits(v[2]) | (f16_bits(v[3]) << 16)};
    *reinterpret_cast<uint2*>(static_cast<unsigned short*>(p) + i) = f16 ? h : b;
  }
}

// Activations from the hardware exp2 / log2 / reciprocal (v_exp_f32,
// v_log_f32, v_rcp_f32); formulas are the textbook ones.
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sigmoidf_(float x) { return frcp(1.0f + fexp(-x)); }
__device__ __forceinline__ float tanhf_(float x) {
  // tanh x = 1 - 2 / (exp(2x) + 1); symmetric form keeps large |x| exact.
  float e = fexp(2.0f * fabsf(x));
  float r = 1.0f - 2.0f * frcp(e + 1.0f);
  return copysignf(r, x);
}
__device__ __forceinline__ float logsigmoidf_(float x) {
  // log sigma(x) = min(x, 0) - log1p(exp(-|x|))
  float e = fexp(-fabsf(x));
  return fminf(x, 0.0f) - __builtin_amdgcn_logf(1.0f + e) * 0.6931471805599453f;
}

// ------------------------------------------------------------------- MFMA
// One 16x16 output tile, K = 32 per call. Both operand layouts put 8
// consecutive logical k in each lane (lane l: row/col l%16, k-block l/16);
// the bf16 instruction consumes that directly, the f32 path issues eight
// 16x16x4 steps over the same k's. Output: lane l, reg i = (row 4*(l/16)+i, col l%16).
template <int MMA> struct Frag;
template <> struct Frag<MMA_BF16> {
  bf16x8 v;
  __device__ __forceinline__ void zero() { v = bf16x8{}; }
};
template <> struct Frag<MMA_F16> {
  f16x8 v;
  __device__ __forceinline__ void zero() { v = f16x8{}; }
};
template <> struct Frag<MMA_F32> {
  float v[8];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.f;
  }
};

// The B operand passes through an empty asm so the optimizer cannot see that
// it is zero in some lanes: the MFMA mixes lanes, yet a "zero operand gives C"
// fold applied per lane would otherwise let the product be skipped or moved
// into code that runs with only part of the wave active.
__device__ __forceinline__ f32x4 mma(const Frag<MMA_BF16>& a, const Frag<MMA_BF16>& b, f32x4 c) {
  bf16x8 bv = b.v;
  asm("" : "+v"(bv));
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, bv, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(const Frag<MMA_F16>& a, const Frag<MMA_F16>& b, f32x4 c) {
  f16x8 bv = b.v;
  asm("" : "+v"(bv));
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, bv, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(const Frag<MMA_F32>& a, const Frag<MMA_F32>& b, f32x4 c) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float bv = b.v[i];
    asm("" : "+v"(bv));
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[i], bv, c, 0, 0, 0);
  }
  return c;
}

// Set fragment element j from an FP32 value (rounded for the bf16 path).
__device__ __forceinline__ void frag_set(Frag<MMA_BF16>& f, int j, float x) {
  f.v[j] = __builtin_bit_cast(__bf16, (unsigned short)bf16_bits(x));
}
__device__ __forceinline__ void frag_set(Frag<MMA_F16>& f, int j, float x) { f.v[j] = (_Float16)x; }
__device__ __forceinline__ void frag_set(Frag<MMA_F32>& f, int j, float x) { f.v[j] = x; }
// Element j of a 16-bit fragment from its raw bits.
__device__ __forceinline__ void frag_bits(Frag<MMA_BF16>& f, int j, uint32_t b) {
  f.v[j] = __builtin_bit_cast(__bf16, (unsigned short)b);
}
__device__ __forceinline__ void frag_bits(Frag<MMA_F16>& f, int j, uint32_t b) {
  f.v[j] = __builtin_bit_cast(_Float16, (unsigned short)b);
}
// Operand rounding of the 16-bit family, and its element bits.
template <int MMA>
__device__ __forceinline__ float round_op(float x) {
  if constexpr (MMA == MMA_BF16) return round_bf16(x);
  else if constexpr (MMA == MMA_F16) return round_f16(x);
  else return x;
}
template <int MMA>
__device__ __forceinline__ uint32_t op_bits(float x) {
  if constexpr (MMA == MMA_F16) return f16_bits(x);
  else return bf16_bits(x);
}

// Rotate a fragment by 8 lanes within each 16-lane row (DPP row_ror:8):
// lane l receives lane l^8's value.
__device__ __forceinline__ int rot8(int v) { return __builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, false); }
__device__ __forceinline__ Frag<MMA_BF16> frag_rot8(const Frag<MMA_BF16>& f) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 v = __builtin_bit_cast(i32x4, f.v);
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = rot8(v[i]);
  Frag<MMA_BF16> o;
  o.v = __builtin_bit_cast(bf16x8, v);
  return o;
}
__device__ __forceinline__ Frag<MMA_F16> frag_rot8(const Frag<MMA_F16>& f) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  i32x4 v = __builtin_bit_cast(i32x4, f.v);
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = rot8(v[i]);
  Frag<MMA_F16> o;
  o.v = __builtin_bit_cast(f16x8, v);
  return o;
}
__device__ __forceinline__ Frag<MMA_F32> frag_rot8(const Frag<MMA_F32>& f) {
  Frag<MMA_F32> o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o.v[i] = __builtin_bit_cast(float, rot8(__builtin_bit_cast(int, f.v[i])));
  return o;
}
template <int MMA>
__device__ __forceinline__ Frag<MMA> frag_sel(bool c, const Frag<MMA>& a, const Frag<MMA>& b) {
  return c ? a : b;
}
template <int MMA>
__device__ __forceinline__ Frag<MMA> frag_keep(bool keep, const Frag<MMA>& f) {
  Frag<MMA> z;
  z.zero();
  return keep ? f : z;
}

// ------------------------------------------------------ exchange words
// 16-bit paths: 32-bit word = (tag << 16) | bf16 or fp16 bits.   F32 path: 64-bit word = (tag << 32) | f32 bits.
// Split words (the BF16 path's backward, whose exchanged gate cotangents are not
// rounded to BF16 by the reference's policy): 32-bit word = the FP32 value rounded
// to 21 mantissa bits, with the tag in the two lowest bits; the reader splits it
// into hi + lo BF16 operands (16 significant bits) and multiplies both.
// Tags cycle 1,1,2,2,1,1,... so a slot (double-buffered by step parity)
// never holds its own step's tag before the step is written, and the
// zero-cleared buffer never matches.
__device__ __forceinline__ uint32_t step_tag(int it) { return 1u + ((uint32_t)(it >> 1) & 1u); }

template <int MMA> struct Word;
template <> struct Word<MMA_BF16> { typedef uint32_t type; };
template <> struct Word<MMA_F16> { typedef uint32_t type; };
template <> struct Word<MMA_F32> { typedef uint64_t type; };

struct Xchg {
  __amdgpu_buffer_rsrc_t rsrc;  // whole exchange region, for the sc1 loads
  char* base;
  int shared_xcd;               // 1: stores write through to memory-side coherence (sc1)
};

__device__ __forceinline__ uint32_t split_word(float v, uint32_t tag) { return ((f2u(v) + 2u) & ~3u) | tag; }

// The exchange region is global memory: say so to the compiler, so the stores
// stay global ones (a flat store would also count in lgkmcnt) even when the
// base pointer has been moved to VGPRs.
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gptr(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

// Store one exchange word. Same-XCD mode uses a non-temporal store (it lands
// in the shared L2); the placement-free mode uses an agent-scope store.
template <int MMA, bool SPLIT = false>
__device__ __forceinline__ void xstore(const Xchg& x, long word, float v, uint32_t tag) {
  if constexpr (MMA != MMA_F32) {
    uint32_t w = SPLIT ? split_word(v, tag) : ((tag << 16) | op_bits<MMA>(v));
    uint32_t* p = reinterpret_cast<uint32_t*>(x.base) + word;
    if (x.shared_xcd) __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else __builtin_nontemporal_store(w, gptr(p));
  } else {
    uint64_t w = ((uint64_t)tag << 32) | f2u(v);
    uint64_t* p = reinterpret_cast<uint64_t*>(x.base) + word;
    if (x.shared_xcd) __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else __builtin_nontemporal_store(w, gptr(p));
  }
}

// Store the NV exchange words of one element (its gates, contiguous) with one
// vector store.
template <int MMA, int NV, bool SPLIT = false>
__device__ __forceinline__ void xstore_vec(const Xchg& x, long word, const float* v, uint32_t tag) {
  if constexpr (MMA != MMA_F32 && NV == 4) {
    typedef uint32_t vec_t __attribute__((ext_vector_type(NV)));
    vec_t w;
#pragma unroll
    for (int i = 0; i < NV; ++i) w[i] = SPLIT ? split_word(v[i], tag) : ((tag << 16) | op_bits<MMA>(v[i]));
    uint32_t* p = reinterpret_cast<uint32_t*>(x.base) + word;
    if (x.shared_xcd) {
#pragma unroll
      for (int i = 0; i < NV; ++i) __hip_atomic_store(p + i, w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      __builtin_nontemporal_store(w, gptr(reinterpret_cast<vec_t*>(p)));
    }
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i) xstore<MMA, SPLIT>(x, word + i, v[i], tag);
  }
}

// Exchange layout of one group's table (BS rows x K words, K = D forward,
// GR*D backward): a run is the 8 consecutive k of one row that one MFMA
// operand lane consumes; it is split into 16-byte chunks (4 words in the BF16
// path, 2 in the FP32 path) and chunk c of every row of run (kt, kq) is
// stored next to the same chunk of the other rows:
//   word(r, k) = (((kt * 4 + kq) * NC + c) * BS + r) * WP + e,
//   kt = k / 32, kq = (k % 32) / 8, c = (k % 8) / WP, e = k % WP.
// Operand lanes hold consecutive rows, so every 16-byte load of a poll reads
// whole 128-byte lines: the address unit handles one line per 8 lanes, not one
// line per lane as with a [row][k] table (2.4x slower for the same bytes).
template <int MMA> struct XLayout {
  static constexpr int WP = MMA == MMA_F32 ? 2 : 4;  // words per 16-byte chunk
  static constexpr int NC = 8 / WP;                   // chunks per run
};
template <int MMA>
__device__ __forceinline__ int xword_of(int BS, int r, int k) {
  return xword_rt(XLayout<MMA>::WP, BS, r, k);
}

// Issue the loads of one 8-word run (8 consecutive k) whose first chunk is at
// word index `word`; its other chunks follow `cstride` bytes apart (16 * BS).
// sc1 (aux 16) makes the load miss the CU-local L1 and read the L2.
template <int MMA> struct Run {  // 16-bit paths
  u32x4 q[2];
  __device__ __forceinline__ void zero() { q[0] = q[1] = u32x4{0u, 0u, 0u, 0u}; }
};
template <> struct Run<MMA_F32> {
  u32x4 q[4];
  __device__ __forceinline__ void zero() { q[0] = q[1] = q[2] = q[3] = u32x4{0u, 0u, 0u, 0u}; }
};

template <int MMA>
__device__ __forceinline__ void xload(const Xchg& x, int word, int cstride, Run<MMA>& r) {
  constexpr int NQ = XLayout<MMA>::NC;
  const int byte = word * (MMA == MMA_F32 ? 8 : 4);
#pragma unroll
  for (int q = 0; q < NQ; ++q) r.q[q] = __builtin_amdgcn_raw_buffer_load_b128(x.rsrc, byte + cstride * q, 0, 16);
}

// Check the tags of a run and unpack it into a fragment.
template <int MMA>
__device__ __forceinline__ bool xunpack(const Run<MMA>& r, uint32_t tag, Frag<MMA>& f) {
  bool ok = true;
  if constexpr (MMA != MMA_F32) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t w = r.q[q][e];
        ok &= (w >> 16) == tag;
        frag_bits(f, 4 * q + e, w & 0xffffu);
      }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        ok &= r.q[q][2 * e + 1] == tag;
        f.v[2 * q + e] = u2f(r.q[q][2 * e]);
      }
  }
  return ok;
}

// Split words (BF16 path only): check the tags of a run and unpack it into
// hi and lo operand fragments: hi = the upper 16 bits of the word (the value
// truncated to BF16), lo = the exact remainder rounded to BF16, so hi + lo is
// the value to about 16 significant bits (the tag bits add < 2^-20 relative).
// Per pair of words: one byte permute (hi), two masks and subtractions and one
// packed conversion (lo); the tags of the 8 words are checked together: every
// word's low two bits equal tag iff both their OR and their AND do.
//
// FP16: hi = the value converted with round-toward-zero (one packed conversion
// per pair), lo = the exact remainder converted the same way: about 22
// significant bits, within FP16's exponent range.
template <int MMA>
__device__ __forceinline__ bool xunpack_split(const Run<MMA>& r, uint32_t tag, Frag<MMA>& hi, Frag<MMA>& lo) {
  static_assert(MMA != MMA_F32, "split words exist on the 16-bit paths only");
  if constexpr (MMA == MMA_F16) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    typedef __fp16 fp16x2_t __attribute__((ext_vector_type(2)));
    uint32_t orv = 0u, andv = ~0u;
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const uint32_t w0 = r.q[q][e], w1 = r.q[q][e + 1];
        const float v0 = u2f(w0 & ~3u), v1 = u2f(w1 & ~3u);
        const f16x2_t h = __builtin_bit_cast(f16x2_t, (fp16x2_t)__builtin_amdgcn_cvt_pkrtz(v0, v1));
        const f16x2_t l =
            __builtin_bit_cast(f16x2_t, (fp16x2_t)__builtin_amdgcn_cvt_pkrtz(v0 - (float)h[0], v1 - (float)h[1]));
        hi.v[4 * q + e] = h[0];
        hi.v[4 * q + e + 1] = h[1];
        lo.v[4 * q + e] = l[0];
        lo.v[4 * q + e + 1] = l[1];
        orv |= w0 | w1;
        andv &= w0 & w1;
      }
    return ((orv & 3u) == tag) & ((andv & 3u) == tag);
  } else {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    u32x4_t hp, lp;
    uint32_t orv = 0u, andv = ~0u;
  #pragma unroll
    for (int q = 0; q < 2; ++q)
  #pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const uint32_t w0 = r.q[q][e], w1 = r.q[q][e + 1];
        hp[2 * q + e / 2] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
        const float l0 = u2f(w0) - u2f(w0 & 0xffff0000u);
        const float l1 = u2f(w1) - u2f(w1 & 0xffff0000u);
        const bf16x2_t l = {(__bf16)l0, (__bf16)l1};
        lp[2 * q + e / 2] = __builtin_bit_cast(uint32_t, l);
        orv |= w0 | w1;
        andv &= w0 & w1;
      }
    hi.v = __builtin_bit_cast(bf16x8, hp);
    lo.v = __builtin_bit_cast(bf16x8, lp);
    return ((orv & 3u) == tag) & ((andv & 3u) == tag);
  }
}

// Unpack a run into the operand(s) of its product: one fragment, or with split
// words the hi and lo fragments.
template <int MMA, bool SPLIT>
struct Operand {
  Frag<MMA> hi, lo;
  __device__ __forceinline__ bool unpack(const Run<MMA>& r, uint32_t tag) {
    if constexpr (SPLIT) return xunpack_split<MMA>(r, tag, hi, lo);
    else return xunpack<MMA>(r, tag, hi);
  }
  // the tags alone (every word's tag equals `tag` iff the OR and the AND of the
  // tag fields both do)
  static __device__ __forceinline__ bool fresh(const Run<MMA>& r, uint32_t tag) {
    if constexpr (MMA != MMA_F32) {
      uint32_t orv = 0u, andv = ~0u;
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          orv |= r.q[q][e];
          andv &= r.q[q][e];
        }
      if constexpr (SPLIT) return ((orv & 3u) == tag) & ((andv & 3u) == tag);
      else return ((orv >> 16) == tag) & ((andv >> 16) == tag);
    } else {
      bool ok = true;
#pragma unroll
      for (int q = 0; q < 4; ++q) ok &= (r.q[q][1] == tag) & (r.q[q][3] == tag);
      return ok;
    }
  }
  __device__ __forceinline__ void keep(bool k) {
    hi = frag_keep<MMA>(k, hi);
    if constexpr (SPLIT) lo = frag_keep<MMA>(k, lo);
  }
  __device__ __forceinline__ Operand rot8() const {
    Operand o;
    o.hi = frag_rot8(hi);
    if constexpr (SPLIT) o.lo = frag_rot8(lo);
    return o;
  }
  // p(frag, part) adds one product into the caller's accumulators (part 1: the lo operand)
  template <typename P>
  __device__ __forceinline__ void apply(P p) const {
    p(hi, 0);
    if constexpr (SPLIT) p(lo, 1);
  }
};

__device__ __forceinline__ uint32_t load_status(const uint32_t* status) {
  return __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_status(uint32_t* status, uint32_t code) {
  atomicMax(status, code);
}

// Workgroup barrier that orders LDS only. __syncthreads() also waits for
// every outstanding global load and store of the wave (vmcnt(0)), which would
// make the I/O waves wait for the HBM loads they issue steps ahead; the
// recurrence kernels exchange data between waves through LDS only, and wait
// for their own global loads explicitly where they need them.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt that waits until at most n vector-memory operations of this wave
// are outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and
// lgkmcnt left at their maxima, i.e. not waited for).
template <int n>
__device__ __forceinline__ void wait_vm() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xf;
}

}  // namespace frnn

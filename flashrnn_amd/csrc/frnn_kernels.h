// Kernel argument blocks and kernel lookup, shared by the kernels and the launcher.
#pragma once

#include <stdint.h>

#include "frnn_plan.h"

namespace frnn {

struct FwdArgs {
  Plan p;
  const void* wx;
  const void* R;
  const void* bias;
  const void* s0;
  void* states;
  void* carry;
  float* save;              // lane-native saved values (training) or null
  void* hsave;              // h_{t-1} copy for the dR GEMM (bf16 or f32 per mma; training) or null
  char* xbuf;               // exchange, both parities
  long long xbytes;
  uint32_t* status;
  uint32_t spin_limit;
};

struct BwdArgs {
  Plan p;
  const void* R;
  const float* save;
  const void* d_states;     // may be null
  const void* d_carry;      // may be null
  void* dwx;
  void* ds0;
  void* dgsave;             // dG copy for the dR GEMM (bf16 or f32 per mma)
  float* dbpart;
  char* xbuf;
  long long xbytes;
  uint32_t* status;
  uint32_t spin_limit;
};

struct GemmArgs {
  Plan p;
  const void* dgsave;
  const void* hsave;
  float* part;
  const float* dbpart;
  void* dR;
  void* db;
};

// Persistent recurrence kernel for (mma, k-tiles per wave) of one cell; null if not built.
const void* lstm_kernel(int mma, int ktw, bool forward);
const void* gru_kernel(int mma, int ktw, bool forward);
const void* elman_kernel(int mma, int ktw, bool forward);
const void* slstm_kernel(int mma, int ktw, bool forward);

inline const void* recurrence_kernel(int cell, int mma, int ktw, bool forward) {
  switch (cell) {
    case 0: return lstm_kernel(mma, ktw, forward);
    case 1: return gru_kernel(mma, ktw, forward);
    case 2: return elman_kernel(mma, ktw, forward);
    case 3: return slstm_kernel(mma, ktw, forward);
  }
  return nullptr;
}
const void* gemm_kernel(int mma);
const void* reduce_kernel();
const void* zero_kernel();

}  // namespace frnn

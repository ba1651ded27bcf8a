/* frnn.h -- C ABI of the MI355X (gfx950) fused recurrent forward/backward library.
 *
 * The library (libfrnn.so) implements the fused multi-head recurrence of
 * FlashRNN: per step g_t = R . h_{t-1} + Wx_t + b, s_t = P(s_{t-1}, g_t), for
 * the LSTM, GRU, Elman and sLSTM cells, forward and backward, on one GPU.
 *
 * It replaces the reference's native boundary, the pybind class
 * FlashRNNFuncFused (flashrnn/flashrnn/fused/flashrnn.cc:244-535):
 *   .forward(training, x, s0, R, b)             (flashrnn.cc:257-333) -> frnn_fwd
 *   .backward(R_t, b, s, g_r, g_i, ds_new)      (flashrnn.cc:335-435) -> frnn_bwd
 * and its host launchers ForwardPass::Run / BackwardPass::Run
 * (fused/flashrnn_fused_forward.cu:773-976, fused/flashrnn_fused_backward.cu:769-1087).
 *
 * Differences of contract, on purpose:
 *  - tensors use the public layouts of flashrnn() (flashrnn/flashrnn/flashrnn.py:1117-1138)
 *    directly, so the caller makes no permuted copies:
 *      Wx [B,T,G_W,N,D]  R [G_R,N,D(out),D(in)]  b [G_T,N,D]
 *      s0 [S,B,N,D] (the [S,B,1,N,D] initial state)  states [S,B,T,N,D]
 *      carry [S,B,N,D] -- the last state in full FP32 (chunk continuation);
 *  - shapes and dtypes are runtime arguments (no JIT, no per-shape build);
 *  - the caller owns every buffer (inputs, outputs, the saved-for-backward
 *    area and the workspace); the library never allocates and never
 *    synchronises; all work is enqueued on the caller's stream;
 *  - errors: a negative return for anything detected on the host; a device
 *    status word (first 4 bytes of the workspace) for anything detected while
 *    the kernels run (a recurrence-exchange timeout, a workgroup placement
 *    that breaks the exchange protocol). frnn_status() reads it.
 *
 * Thread safety: frnn_cell_sizes, frnn_workspace_bytes, frnn_fwd, frnn_fwd_projected, frnn_bwd,
 * frnn_status and frnn_strerror keep no state between calls and may run from
 * several threads at once; calls that overlap in time must use distinct
 * workspaces. The tuning, test and profiling setters (frnn_set_spin_limit,
 * frnn_set_scouts, frnn_set_gemm_dma, frnn_timing_enable/_read,
 * frnn_set_phase_profile) change process-global settings that every later
 * call reads, on every thread: set them while no other thread is calling.
 * frnn_set_gemm_dma also changes frnn_workspace_bytes(d, 1), so size the
 * backward workspace after setting it.
 */
#ifndef FRNN_H
#define FRNN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* frnn_stream_t; /* == hipStream_t */

enum frnn_cell { FRNN_LSTM = 0, FRNN_GRU = 1, FRNN_ELMAN = 2, FRNN_SLSTM = 3 };
enum frnn_dtype { FRNN_F32 = 0, FRNN_BF16 = 1, FRNN_F16 = 2 };
/* Recurrent-product arithmetic:
 *  FRNN_MMA_BF16: R and h_{t-1} rounded to BF16, FP32 accumulation, FP32
 *    state and pointwise -- the reference's numerics="fp32_state_bf16_mma"
 *    (flashrnn/flashrnn2/torch_backend.py:21-35). Backward rounds the
 *    recurrent cotangents through BF16 the same way.
 *  FRNN_MMA_F32: FP32 operands and accumulation -- numerics="mathematical" in FP32.
 *  FRNN_MMA_F16: as FRNN_MMA_BF16 with FP16 operands: FlashRNN2's FP16 contract (FP16
 *    inputs, FP32 compute and state; flashrnn/flashrnn2/state_contract.py:21-49). */
enum frnn_mma { FRNN_MMA_BF16 = 0, FRNN_MMA_F32 = 1, FRNN_MMA_F16 = 2 };
enum frnn_flags {
  FRNN_TRAINING = 1,       /* frnn_fwd fills the saved-for-backward area */
  FRNN_XCD_SHARED = 2,     /* exchange through memory-side coherence (slower; any placement) */
  /* The reference's FlashRNNConfig.gradient_recurrent_cut (flashrnn/flashrnn/flashrnn.py:129,
   * 784-787; fused/flashrnn_fused_backward_cut.cu): frnn_bwd passes no R^T dG cotangent
   * to h_{t-1}; direct paths, dR and db are unchanged. */
  FRNN_GRAD_CUT = 4,
  /* The reference's gradient_recurrent_clipval = clipval (flashrnn.py:131, 357-380): frnn_fwd
   * clamps each new hidden state to [-clipval, clipval] (the fused build passes the same value
   * as its forward clip value, flashrnn.py:368-372; the backward passes straight through the
   * clamp), and frnn_bwd clamps the recurrent cotangent of h_{t-1} (direct path plus R^T dG)
   * to the same interval before adding the caller's cotangent
   * (fused/lstm_fused_pointwise.cuh:76-80, 115-124). */
  FRNN_GRAD_CLIP = 8,
  /* Tests of failure handling only: every exchange poll waits for a tag that is never
   * written, so each wait ends at the spin limit (frnn_set_spin_limit) with FRNN_E_TIMEOUT
   * and every wave leaves its loop. */
  FRNN_TEST_UNREADY = 16,
  /* Output policies of FlashRNN2's prepared and training calls
   * (flashrnn/flashrnn2/prepared.py:18-71, triton_persistent.py:154-166, training.py:91-124).
   * FRNN_OUT_HIDDEN: states_out is the hidden-state history only, [B,T,N,D]; for
   * frnn_bwd, states is that history and d_states is its cotangent, [B,T,N,D].
   * FRNN_OUT_LAST (forward only, not with FRNN_TRAINING): states_out is the hidden
   * state of the sequence's last step only, [B,1,N,D], written by the call whose
   * window ends the sequence. FRNN_SNAPSHOT_F32: states_out (and, for frnn_bwd,
   * states and d_states) are FP32 instead of dtype_io. A backward passes the flags of
   * its training forward. */
  FRNN_OUT_HIDDEN = 32,
  FRNN_OUT_LAST = 64,
  FRNN_SNAPSHOT_F32 = 128,
  /* sLSTM backward under the FlashRNN v1 gradient convention, which FlashRNN2's training
   * keeps (flashrnn/flashrnn2/grad_reference.py:1-12, vanilla_fwbw/bw.py): the stabilizer
   * m carries no cotangent (so the initial m's is zero) and the normalizer clamp
   * max(n, 1) passes its cotangent straight through. Without it the backward is the
   * exact gradient of flashrnn_torch (flashrnn2/reference.py:98-112). Other cells ignore it. */
  FRNN_SLSTM_V1GRAD = 256,
};

typedef struct frnn_desc {
  int32_t cell;        /* enum frnn_cell */
  int32_t batch;       /* B */
  int32_t steps;       /* T */
  int32_t heads;       /* N */
  int32_t width;       /* D, multiple of 32, <= 1024 */
  int32_t dtype_io;    /* dtype of Wx, R, b, states, dWx, dR, db, d_states */
  int32_t dtype_state; /* dtype of s0, ds0, carry and d_carry */
  int32_t mma;         /* enum frnn_mma */
  int32_t flags;       /* enum frnn_flags */
  float clipval;       /* with FRNN_GRAD_CLIP: finite and >= 0; otherwise ignored */
  /* Forward step window (FlashRNN2's chunked prepared execution, prepared.py:114-162):
   * Wx and states_out hold total_steps steps, and the call runs steps
   * [step_base, step_base + steps) of them from s0, writing those steps of
   * states_out in place. total_steps == 0 means steps. The sLSTM zero-normalizer
   * predicate applies only at step 0 of the sequence (step_base == 0). Not with
   * FRNN_TRAINING (the backward needs a whole sequence). */
  int32_t total_steps;
  int32_t step_base;
} frnn_desc;

enum frnn_status {
  FRNN_OK = 0,
  FRNN_E_INVALID = -1,     /* null pointer, bad enum, bad shape */
  FRNN_E_UNSUPPORTED = -2, /* valid but not implemented (e.g. width not a multiple of 32) */
  FRNN_E_WORKSPACE = -3,   /* workspace smaller than frnn_workspace_bytes() */
  FRNN_E_LAUNCH = -4,      /* the HIP runtime refused a launch (co-residency, resources) */
  FRNN_E_TIMEOUT = -5,     /* device: a recurrence exchange did not arrive within the spin limit */
  FRNN_E_PLACEMENT = -6,   /* device: an XCD received more workgroups than it has slots */
  FRNN_E_SCRATCH = -7,     /* frnn_fwd_noalloc: the forward workspace exceeds its static scratch */
};

/* Gate and state counts of a cell: (G_R, G_W, G_T, S); flashrnn/flashrnn/flashrnn.py:45-70. */
int frnn_cell_sizes(int cell, int32_t* g_r, int32_t* g_w, int32_t* g_t, int32_t* s);

/* Bytes of the caller-owned areas. which: 0 = forward workspace,
 * 1 = backward workspace, 2 = saved-for-backward area (written by a training
 * forward, read by the matching backward), 3 = workspace of frnn_fwd_projected.
 * Returns 0 for an invalid desc. */
size_t frnn_workspace_bytes(const frnn_desc* d, int which);

/* Forward. Replaces FlashRNNFuncFused::forward (fused/flashrnn.cc:257-333).
 * states_out: [S,B,T,N,D] in dtype_io, or what the output-policy flags select
 * (FRNN_OUT_HIDDEN, FRNN_OUT_LAST, FRNN_SNAPSHOT_F32; T = total_steps with a step
 * window). carry_out: [S,B,N,D] in dtype_state (may be NULL). save: the
 * saved-for-backward area (may be NULL unless FRNN_TRAINING). */
int frnn_fwd(const frnn_desc* d, const void* wx, const void* R, const void* b, const void* s0,
             void* states_out, void* carry_out, void* save, void* ws, size_t ws_bytes,
             frnn_stream_t stream);

/* Input projection and forward in one call. Replaces the layer around the reference's
 * recurrence: TorchLayer (flashrnn/flashrnn2/torch_layer.py:14-80) runs Wx = x W^T as a
 * separate library GEMM, then the recurrence (README.md:17 leaves the projection to the
 * caller). Here the projection's workgroups run on the CUs the recurrence leaves free, in
 * the same launch, and the recurrence reads each step's Wx rows as soon as they are
 * written; where the recurrence needs the whole GPU (or successive launches) the
 * projection runs in a launch of its own first. Results equal frnn_fwd on the Wx this
 * call writes, bitwise, either way.
 * x [B,T,input_size] and w_in [G_W,N,D,input_size] in dtype_io, which must be the MMA's
 * 16-bit type (BF16 with FRNN_MMA_BF16, FP16 with FRNN_MMA_F16); input_size a multiple
 * of 8; x, w_in and wx_out 16-byte aligned. wx_out [B,T,G_W,N,D] (dtype_io) receives
 * the projection (FP32 accumulation, rounded once). Whole sequences only (no step
 * window). ws: frnn_workspace_bytes(d, 3) bytes. Other arguments as frnn_fwd. */
int frnn_fwd_projected(const frnn_desc* d, int32_t input_size, const void* x, const void* w_in, void* wx_out,
                       const void* R, const void* b, const void* s0, void* states_out, void* carry_out,
                       void* save, void* ws, size_t ws_bytes, frnn_stream_t stream);

/* Allocation-free forward. No counterpart in the reference: it is for callers that
 * cannot allocate device memory, or have a library do so, around the call -- code under
 * HIP graph capture, tight serving loops, harnesses that forbid it.
 * Same arguments, results and kernels as frnn_fwd, except that the forward workspace
 * (exchange tables and workgroup slot counters) lives in a static device array of the
 * library, 8 MiB per GPU, held by each GPU it runs on until the process ends; the call
 * makes no hipMalloc, hipFree or allocating library call. status: a caller-owned device
 * word (4 bytes, zeroed once by the caller) that receives the sticky device status, as
 * the first word of frnn_fwd's workspace does (frnn_status(status, stream) reads it).
 * Returns FRNN_E_SCRATCH when frnn_workspace_bytes(d, 0) exceeds 8 MiB (about
 * groups * D <= 32768 with 16-bit operands, 16384 with FP32, groups = N * ceil(B/16)).
 * Every call on one GPU shares that GPU's array, and the array keeps the last call's
 * contents (each call clears what must start at zero): calls that overlap in time on
 * one GPU race -- serialise them on one stream. save is the caller's area, as in
 * frnn_fwd (may be NULL unless FRNN_TRAINING). */
int frnn_fwd_noalloc(const frnn_desc* d, const void* wx, const void* R, const void* b, const void* s0,
                     void* states_out, void* carry_out, void* save, void* status, frnn_stream_t stream);

/* Backward. Replaces FlashRNNFuncFused::backward (fused/flashrnn.cc:335-435).
 * R, s0, states (the forward's states_out) and save must be those of the
 * training forward, and d carries its flags. d_states: [S,B,T,N,D] (dtype_io;
 * [B,T,N,D] with FRNN_OUT_HIDDEN, FP32 with FRNN_SNAPSHOT_F32; may be NULL = zero);
 * d_carry: [S,B,N,D] (dtype_state, may be NULL = zero). Outputs dwx
 * [B,T,G_W,N,D], dR [G_R,N,D,D], db [G_T,N,D] (dtype_io) and ds0 [S,B,N,D]
 * (dtype_state) are overwritten. */
int frnn_bwd(const frnn_desc* d, const void* R, const void* s0, const void* states, const void* save,
             const void* d_states, const void* d_carry, void* dwx, void* dR, void* db, void* ds0,
             void* ws, size_t ws_bytes, frnn_stream_t stream);

/* Waits for the stream, then returns the device status word of ws
 * (FRNN_OK, FRNN_E_TIMEOUT, FRNN_E_PLACEMENT). */
int frnn_status(const void* ws, frnn_stream_t stream);

/* Static description of an error code. */
const char* frnn_strerror(int code);

/* Optional kernel timing. When enabled, every persistent forward recurrence,
 * backward recurrence and dR GEMM (+ its reduction) launch is bracketed by a
 * pair of HIP events on the caller's stream (events owned by the library).
 * frnn_timing_read() waits for the recorded events, returns the summed
 * milliseconds and launch counts per kind -- [0] forward recurrence,
 * [1] backward recurrence, [2] dR GEMM + reduction -- and clears the record.
 * Not reentrant: a profiling aid for one thread. */
void frnn_timing_enable(int on);
int frnn_timing_read(double* ms3, int32_t* counts3);

/* Optional phase profile (a profiling aid): when set to a device buffer of
 * 256 zeroed 64-bit words, every wave of workgroup 0 accumulates cycle counts
 * of its time loop into 8 words of its own (wave w at 8*w; forward kernel in
 * words 0-127, backward in 128-255). Compute waves: [0] exchange wait,
 * [1] MFMA and LDS partials, [2] workgroup barrier, [3] cell arithmetic,
 * [4] exchange polls, [5] steps, [6] backward partial-sum reduction. I/O
 * waves: [0] ring fill, [1] load issue, [2] barrier, [3] output drain,
 * [5] steps. Every wave of workgroups 0-127 also writes a timeline of steps
 * 64-71 (eight 100 MHz clock stamps per step, 64 words per wave) at word
 * 256 + (workgroup * 16 + wave) * 64 (forward) and 131328 + the same
 * (backward); the buffer then needs 262400 words. NULL disables. */
void frnn_set_phase_profile(void* device_words);

/* Test hook: the spin limit of the exchange waits (default 1<<22 polls; 0 restores it).
 * A tiny value forces FRNN_E_TIMEOUT from the host without faulting. */
void frnn_set_spin_limit(uint32_t polls);

/* Tuning hook, no counterpart in the reference: enable (1, the default unless the
 * environment sets FRNN_NO_SCOUT=1) or disable (0) the backward's scouts, one extra
 * workgroup per group that pulls the inputs of later steps into the L2 of the group's
 * XCD. They change timing only, never results; they are used only where they cost no
 * extra launch and get a CU to themselves. */
void frnn_set_scouts(int enable);

/* Tuning hook, no counterpart in the reference: enable (1, the default unless the
 * environment sets FRNN_NO_GEMM_DMA=1) or disable (0) the dR GEMM whose operand tiles
 * are loaded by LDS-DMA (used for 16-bit operands already in the MMA type and D % 64 == 0,
 * every cell; the GRU's FP32 candidate-gate cotangents and an FP32 s0 are first rounded
 * to 16-bit copies in the backward workspace). Both kernels give bitwise the same dR. */
void frnn_set_gemm_dma(int enable);

#ifdef __cplusplus
}
#endif
#endif /* FRNN_H */

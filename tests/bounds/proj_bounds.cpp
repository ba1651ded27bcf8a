// Host bounds check of the input projection's addressing (CPU only).
//
// For a problem and input size it builds the projection arguments the way
// frnn_fwd_projected does, with the plan libfrnn.so makes (frnn_test_plan) and
// its workspace size (frnn_workspace_bytes(d, 3)), and enumerates, with the
// index functions the workers call (proj_x_row, proj_w_row, proj_k8,
// proj_wx_elem in flashrnn_amd/csrc/frnn_kernels.h), every 16-byte operand
// load of both worker kinds (proj_wave_worker, proj_wg_worker in frnn_proj.h)
// -- including the k runs past I and the rows / columns past the end -- every
// 8-byte Wx store, the readiness counters the workers raise and the forward's
// gate reads, and the LDS offsets of the workgroup worker; each is checked
// against its buffer's extent. The lane -> work mapping mirrors the workers.
//
// Usage: proj_bounds cell B T N D io(1=bf16,2=f16) I
// Prints "violations N"; exit status 1 on any violation.
#include <cstdio>
#include <cstdlib>

#include "../../flashrnn_amd/csrc/frnn_kernels.h"
#include "../../include/frnn.h"

using namespace frnn;

static long long violations = 0, checked = 0;
static void check(const char* what, long long lo, long long hi, long long extent) {
  ++checked;
  if (lo < 0 || hi > extent || lo > hi) {
    if (violations < 10) std::printf("  VIOLATION %s: [%lld, %lld) outside [0, %lld)\n", what, lo, hi, extent);
    ++violations;
  }
}

int main(int argc, char** argv) {
  if (argc != 8) {
    std::fprintf(stderr, "usage: proj_bounds cell B T N D io I\n");
    return 2;
  }
  frnn_desc d = {};
  d.cell = std::atoi(argv[1]);
  d.batch = std::atoi(argv[2]);
  d.steps = std::atoi(argv[3]);
  d.heads = std::atoi(argv[4]);
  d.width = std::atoi(argv[5]);
  d.dtype_io = std::atoi(argv[6]);
  d.dtype_state = FRNN_F32;
  d.mma = d.dtype_io == FRNN_F16 ? FRNN_MMA_F16 : FRNN_MMA_BF16;
  const int I = std::atoi(argv[7]);
  Plan p;
  if (frnn_test_plan(&d, &p, sizeof(p)) != FRNN_OK) return 2;
  const long long ws3 = (long long)frnn_workspace_bytes(&d, 3);
  ProjArgs pa = {};
  pa.I = I;
  pa.ncols = p.GW * p.N * p.D;
  pa.B = p.B;
  pa.T = p.T;
  pa.nrt = (int)(((long long)p.B * p.T + kProjRows - 1) / kProjRows);
  pa.nct = (pa.ncols + kProjCols - 1) / kProjCols;
  const long long rows = (long long)p.B * p.T;
  const long long x_ext = rows * I, w_ext = (long long)pa.ncols * I, wx_ext = rows * pa.ncols;
  // counters after the forward workspace: ready[nrt], then the tile counter
  check("readiness counters", p.ws_fwd, p.ws_fwd + 4LL * (pa.nrt + 1), ws3);
  const int ntiles = pa.nrt * pa.nct;
  for (int tile = 0; tile < ntiles; ++tile) {
    const int rt = tile / pa.nct, ct = tile % pa.nct;
    check("ready[rt]", rt, rt + 1, pa.nrt);
    const int c0 = ct * kProjCols;
    const long long m0 = (long long)rt * kProjRows;
    // ---- workgroup worker: LDS-DMA stages of 64 k
    for (int wv = 0; wv < 4; ++wv)
      for (int lane = 0; lane < 64; ++lane)
        for (int j = 0; j < 4; ++j) {
          const int r = wv * 32 + 8 * j + (lane >> 3), q = ((lane & 7) ^ (r >> 1)) & 7;
          const long a = proj_w_row(pa, c0 + r), b = proj_x_row(pa, m0 + r);
          for (int k0 = 0; k0 < I; k0 += 64) {
            const int k8 = proj_k8(pa, k0 + 8 * q);
            check("wg W load", a + k8, a + k8 + 8, w_ext);
            check("wg x load", b + k8, b + k8 + 8, x_ext);
          }
          check("wg LDS DMA", (wv * 32 + 8 * j) * 128 + 16 * lane, (wv * 32 + 8 * j) * 128 + 16 * lane + 16, 128 * 128);
        }
    for (int r = 0; r < 128; ++r)
      for (int q = 0; q < 8; ++q) {
        const int off = r * 128 + ((q ^ (r >> 1)) & 7) * 16;
        check("wg LDS fragment", off, off + 16, 128 * 128);
      }
    // ---- wave worker: four 64 x 64 quarters, k in steps of 32 (loads run one step past I)
    for (int quarter = 0; quarter < 4; ++quarter)
      for (int lane = 0; lane < 64; ++lane) {
        const int r16 = lane & 15, kq = lane >> 4;
        const int qc0 = c0 + 64 * (quarter & 1);
        const long long qm0 = m0 + 64 * (quarter >> 1);
        for (int i = 0; i < 4; ++i) {
          const long a = proj_w_row(pa, qc0 + 16 * i + r16), b = proj_x_row(pa, qm0 + 16 * i + r16);
          for (int k0 = 0; k0 <= I + 64; k0 += 32) {
            const int k8 = proj_k8(pa, k0 + 8 * kq);
            check("wave W load", a + k8, a + k8 + 8, w_ext);
            check("wave x load", b + k8, b + k8 + 8, x_ext);
          }
        }
      }
    // ---- stores (both workers: 64 x 64 quarters, lane = 4 columns of one row)
    for (int quarter = 0; quarter < 4; ++quarter)
      for (int lane = 0; lane < 64; ++lane)
        for (int jr = 0; jr < 4; ++jr)
          for (int i = 0; i < 4; ++i) {
            const long long m = m0 + 64 * (quarter >> 1) + 16 * jr + (lane & 15);
            const int c = c0 + 64 * (quarter & 1) + 16 * i + 4 * (lane >> 4);
            if (m >= rows || c >= pa.ncols) continue;
            const long e = proj_wx_elem(pa, m, c);
            check("Wx store", e, e + 4, wx_ext);
            if (e % 4) check("Wx store alignment", 1, 0, 0);
          }
  }
  // ---- the forward's gate: row tiles each step reads, counters four at a time
  for (int u = 0; u < p.T; ++u) {
    const int need = proj_last_row_tile(u, p.B);
    check("gate row tile", need, need + 1, pa.nrt);
  }
  std::printf("B%d T%d N%d D%d I%d: %d x %d tiles, %lld accesses checked\nviolations %lld\n", p.B, p.T, p.N, p.D, I,
              pa.nrt, pa.nct, checked, violations);
  return violations ? 1 : 0;
}

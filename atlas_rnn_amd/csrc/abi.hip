// abi.hip - extern "C" entry points of libatlas_mem.so (declared in include/atlas_mem.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/atlas_mem.h"
#include "mem_common.h"
#include "mem_params.h"
#include "seg_common.h"

#include <cstdlib>

namespace atlas {
template <typename T, int CHF, int CHB>
hipError_t launch_chunk_coef_pair(const Geom& gf, const Geom& gb, const T* decay, const T* lr, const T* beta,
                                  const T* gate, float* rec_f, T* wsh_f, float* rec_b, T* wsh_b, hipStream_t stream);
template <typename T, int CH, int D>
hipError_t launch_fwd_seg(const Geom&, const FwdPtrs<T>&, const SegGeom&, float*, float*, float*, float*, float*,
                          T*, hipStream_t);
template <typename T, int CH, int D>
hipError_t launch_bwd_seg(const Geom&, const BwdPtrs<T>&, const SegGeom&, const BwdSegPtrs&, hipStream_t, bool,
                          const AggOverFwd*);
bool walk_fwd_supported(const Geom& g);
bool chunk_coef_fwd_supported(const Geom& g);
hipError_t launch_chunk_coef_fwd(const Geom& g, const bf16* decay, const bf16* lr, const bf16* beta, const bf16* gate,
                                 float* coef, bf16* wsh, hipStream_t stream);
hipError_t launch_buf_state(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, const float* coef, float* corr,
                            hipStream_t stream);
hipError_t launch_buf_y(const Geom& g, const FwdPtrs<bf16>& a, const bf16* wsh, hipStream_t stream);
hipError_t launch_walk_fwd(const Geom& g, const FwdPtrs<bf16>& a, const SegGeom& sg, float* agg, float* seg_states,
                           float* rw, float* final_raw, float* coef, bf16* wsh, hipStream_t stream);
bool chunk_bwd_supported(const Geom& g, const SegGeom& sg);
size_t chunk_bwd_states_bytes(const Geom& g);

// Diagnostic tile product C = A B^T (16 x 64 inputs) through the same fragment helpers.
template <typename T>
__global__ __launch_bounds__(64) void k_mfma_selftest(const T* A, const T* B, float* C) {
  __shared__ __align__(16) T sa[16][64 + 8];
  __shared__ __align__(16) T sb[16][64 + 8];
  const int l = threadIdx.x;
  for (int idx = l; idx < 16 * 64; idx += 64) {
    sa[idx / 64][idx % 64] = A[idx];
    sb[idx / 64][idx % 64] = B[idx];
  }
  __syncthreads();
  typedef MM<T> M;
  f32x4 acc = zero4(), acc2 = zero4();
  for (int k0 = 0; k0 < 64; k0 += M::KS) {
    acc = M::mma(frag_ld_row<T>(&sa[0][0], 64 + 8, 0, k0), frag_ld_row<T>(&sb[0][0], 64 + 8, 0, k0), acc);
    // strided path: read B^T through (rs = 1, cs = row stride) of a transposed view of the same data
    acc2 = M::mma(frag_ld<T>(&sa[0][0], 64 + 8, 1, 0, k0), frag_ld<T>(B, 64, 1, 0, k0), acc2);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * (l >> 4) + r, n = l & 15;
    C[m * 16 + n] = acc[r];
    C[256 + m * 16 + n] = acc2[r];
  }
}
}  // namespace atlas

using namespace atlas;

// ---------------------------------------------------------------------------------------------
// Opt-in kernel timing: when enabled, every launch is bracketed by two HIP events recorded on the
// launch stream; atlas_mem_profile_read() waits for them and accumulates per-kernel time.
// ---------------------------------------------------------------------------------------------
namespace {
struct Pending { int kid; hipEvent_t a, b; };
struct Profiler {
  std::mutex mu;
  bool on = false;
  std::vector<hipEvent_t> pool;
  std::vector<Pending> pending;
  hipEvent_t open[KID_COUNT] = {};
  double ms[KID_COUNT] = {};
  long long n[KID_COUNT] = {};
  hipEvent_t take() {
    if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
Profiler& prof() { static Profiler p; return p; }
// kernel launched last for each timed stage (the specialised and the general path launch different
// kernels for the same stage; prof_name records which)
const char* kKernelNames[KID_COUNT] = {"k_fwd_seg_agg", "k_fwd_seg", "k_buffer_out", "k_bwd_seg_agg",
                                       "k_bwd_seg", "k_bwd_seg_fixup", "k_seg_reduce_dsref", "k_fwd_seg_scan",
                                       "k_bwd_seg_scan", "k_chunk_coef_fwd", "k_chunk_coef_bwd",
                                       "k_bwd_scalar", "k_buf_fwd", "k_buf_bwd"};
}  // namespace

namespace atlas {
void prof_name(int kid, const char* name) {
  if (kid >= 0 && kid < KID_COUNT) kKernelNames[kid] = name;
}
void prof_begin(int kid, hipStream_t s) {
  Profiler& P = prof();
  if (!P.on) return;
  std::lock_guard<std::mutex> lk(P.mu);
  hipEvent_t e = P.take();
  if (!e) return;
  hipEventRecord(e, s);
  P.open[kid] = e;
}
void prof_end(int kid, hipStream_t s) {
  Profiler& P = prof();
  if (!P.on) return;
  std::lock_guard<std::mutex> lk(P.mu);
  hipEvent_t a = P.open[kid];
  if (!a) return;
  hipEvent_t b = P.take();
  if (!b) return;
  hipEventRecord(b, s);
  P.pending.push_back({kid, a, b});
  P.open[kid] = nullptr;
}
}  // namespace atlas

namespace {

struct Plan {
  Geom g;      // forward chunks (Lc <= 64 bf16, 32 fp32)
  SegGeom sg;
  Geom gb;     // backward chunks (Lb <= 32 bf16, 16 fp32; Lb divides Lc)
  SegGeom sgb;
  int CH;      // forward chunk capacity (kernel template), 64 bf16 / 32 fp32
  int CHB;     // backward chunk capacity, 32 bf16 / 16 fp32
  int esize;   // bytes per input element
  bool ok;
  int status;
  // scan_chunk_len clamps at chunk ends: the segment-parallel sequence (this plan, unclamped, checking
  // the clamp points) runs first and the exact one-segment-per-row sequence (make_plan(p, true))
  // runs behind it only when some clamp point's |S| exceeds 100 (the clamp is the identity otherwise)
  bool dual;
  // the specialised forward walk with the backward of chunk_bwd.hip (bf16, d = 64, window <= 17, no
  // clamp, no carried buffer): the forward saves no boundary states and no backward records, and
  // its chunks have no mid point (Lmid = 0)
  bool cbwd;
  // cbwd plans: the forward records formed on the matrix cores (chunk_coef.hip) instead of by the
  // per-source chains (coef.hip)
  bool ccoef;
};

#ifndef ATLAS_CHUNK_BWD
#define ATLAS_CHUNK_BWD 1
#endif
#ifndef ATLAS_CHUNK_COEF
#define ATLAS_CHUNK_COEF 1
#endif

// Segments per head-batch row: enough (segment, bh) workgroups for one per CU (the walks hold a
// CU's LDS, so a second round of workgroups would only queue behind the first); a single segment
// when S is clamped at scan_chunk_len boundaries (not affine). The CU count is MI355X's, fixed so
// that the saved / workspace sizes do not depend on the device queried.
constexpr int kCUs = 256;
SegGeom make_seg(const Geom& g) {
  SegGeom s{};
  int G;
  if (g.clamp_every > 0) {
    G = g.nc;
  } else {
    const int want = g.BH >= kCUs ? 1 : (kCUs + g.BH - 1) / g.BH;
    G = (g.nc + want - 1) / want;
  }
  if (G < 1) G = 1;
  if (G > g.nc) G = g.nc;
  s.G = G;
  s.nseg = (g.nc + G - 1) / G;
  s.agg_stride = 2 * g.DV * g.DK + 16;
  return s;
}

int chunk_cap(int dtype) { return dtype == ATLAS_DT_BF16 ? 64 : 32; }
constexpr int kMinClampChunk = 8;   // shortest backward chunk accepted under clamp_every
int bwd_chunk_cap(int dtype) { return dtype == ATLAS_DT_BF16 ? 32 : 16; }
int largest_divisor_at_most(int n, int cap) {
  for (int d = cap; d >= 1; --d)
    if (n % d == 0) return d;
  return 1;
}

Plan make_plan(const atlas_mem_problem* p, bool serial_clamp = false) {
  Plan pl{};
  pl.ok = false;
  pl.status = ATLAS_MEM_ERR_ARG;
  if (!p) { pl.status = ATLAS_MEM_ERR_NULL; return pl; }
  if (p->abi_version != ATLAS_MEM_ABI_VERSION) { pl.status = ATLAS_MEM_ERR_ABI; return pl; }
  if (p->dtype != ATLAS_DT_F32 && p->dtype != ATLAS_DT_BF16) { pl.status = ATLAS_MEM_ERR_DTYPE; return pl; }
  if (p->bh < 1 || p->seq_len < 1 || p->window < 1 || p->window > kMaxWindow) { pl.status = ATLAS_MEM_ERR_SHAPE; return pl; }
  if (p->d_k != p->d_v || (p->d_k != 32 && p->d_k != 64)) { pl.status = ATLAS_MEM_ERR_SHAPE; return pl; }
  if ((p->momentum != 0 && p->momentum != 1) || p->gate_mode < 0 || p->gate_mode > 2 ||
      p->map_mode < 0 || p->map_mode > 1 || p->map_degree < 1 || p->map_degree > 16 ||
      (p->has_buffer != 0 && p->has_buffer != 1) || p->clamp_every < 0 ||
      (p->clamp_final != 0 && p->clamp_final != 1)) {
    return pl;
  }
  if (p->has_buffer && p->window == 1) return pl;
  const int CH = chunk_cap(p->dtype);
  int Lc = CH;
  if (p->clamp_every > 0 && p->clamp_every % CH != 0) Lc = largest_divisor_at_most(p->clamp_every, CH);
  const int Lb = largest_divisor_at_most(Lc, bwd_chunk_cap(p->dtype));
  // the forward saves the state at every backward-chunk boundary: at most one inside a chunk
  if (Lc / Lb > 2) Lc = Lb;
  const int H = p->window - 1;
  if (Lb < H) { pl.status = ATLAS_MEM_ERR_UNSUPPORTED; return pl; }
  // clamp_every with no divisor of at least kMinClampChunk in range (37, 74, ...) would walk the
  // row in chunks of a few tokens with a state saved after each: the caller splits such calls at
  // clamp_every instead (one unclamped call per scan chunk, state carried)
  if (p->clamp_every > 0 && Lb < kMinClampChunk) { pl.status = ATLAS_MEM_ERR_UNSUPPORTED; return pl; }
  Geom& g = pl.g;
  g.BH = p->bh; g.T = p->seq_len; g.DK = p->d_k; g.DV = p->d_v;
  g.e = p->window; g.H = H; g.Lc = Lc; g.nc = (p->seq_len + Lc - 1) / Lc;
  g.Lmid = Lc / Lb == 2 ? Lb : 0;
  g.ncb = (p->seq_len + Lb - 1) / Lb;
  g.momentum = p->momentum; g.gate_mode = p->gate_mode; g.map_mode = p->map_mode;
  g.map_deg = p->map_mode == ATLAS_MAP_ELEMENTWISE ? p->map_degree : 1;
  g.has_buf = p->has_buffer; g.clamp_every = p->clamp_every; g.clamp_final = p->clamp_final;
  g.flag = nullptr; g.flag_run = -1; g.flag_reset = 0; g.clamp_check = 0;
  // clamp points on forward-chunk ends: segment-parallel with the clamp points checked (dual)
  pl.dual = !serial_clamp && p->clamp_every > 0 && p->clamp_every % CH == 0 && p->clamp_every < p->seq_len;
  if (pl.dual) g.clamp_every = 0;
  pl.sg = make_seg(g);
  pl.cbwd = ATLAS_CHUNK_BWD && p->dtype == ATLAS_DT_BF16 && !pl.dual && walk_fwd_supported(g) &&
            chunk_bwd_supported(g, pl.sg);
  if (pl.cbwd) g.Lmid = 0;
  pl.ccoef = ATLAS_CHUNK_COEF && pl.cbwd && chunk_coef_fwd_supported(g);
  // backward: same segments, chunks of Lb
  Geom& gb = pl.gb;
  gb = g;
  gb.Lc = Lb;
  gb.nc = (p->seq_len + Lb - 1) / Lb;
  gb.Lmid = 0;
  pl.sgb = pl.sg;
  pl.sgb.G = pl.sg.G * (Lc / Lb);
  pl.CH = CH;
  pl.CHB = bwd_chunk_cap(p->dtype);
  pl.esize = p->dtype == ATLAS_DT_BF16 ? 2 : 4;
  pl.ok = true;
  pl.status = ATLAS_MEM_OK;
  return pl;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// `saved` layout: segment-start states, segment aggregates (forward scratch), raw S_{T-1}, the raw
// state at every backward-chunk boundary (written by the forward walk, read by the backward).
struct SavedLayout {
  size_t seg, agg, final_raw, rw, coef, wsh, bcoef, bwsh, bufc, total;
};

// the specialised walks with a carried buffer take its first-chunk terms from bufwalk.hip
bool walk_with_buffer(const Plan& pl) { return pl.esize == 2 && pl.g.has_buf && walk_fwd_supported(pl.g); }

// floats per chunk coefficient record (acoef, kcoef, endc, wsend, wzend, wsmid, wzmid, midc)
size_t coef_rec_floats(int ch) { return (size_t)2 * ch + 8 + 4 * (ch + kHaloPad); }

// floats per backward chunk of the scalar-gradient inputs (ScalarBlock: Lm, hS, hZ, fS, fZ, Grams)
size_t scalar_block_floats(int ch) { return (size_t)ch * (ch + kHaloPad) + 2 * (ch + kHaloPad) + 2 * ch + 4; }

SavedLayout saved_layout(const Plan& pl) {
  const Geom& g = pl.g;
  SavedLayout L{};
  const size_t st = (size_t)g.DV * g.DK * sizeof(float);
  size_t off = 0;
  L.seg = off; off += align256((size_t)g.BH * pl.sg.nseg * 2 * st);
  L.agg = off; off += align256((size_t)g.BH * pl.sg.nseg * pl.sg.agg_stride * sizeof(float));
  L.final_raw = off; off += align256((size_t)g.BH * st);
  // the backward of chunk_bwd.hip takes the states at the 64-token chunk starts and forms its own
  // records; the earlier backward, the states at every backward-chunk boundary and its records
  const bool brec = !pl.cbwd;
  L.rw = off; off += align256(brec ? (size_t)g.BH * g.ncb * 2 * st : chunk_bwd_states_bytes(g));
  // forward scratch: per-chunk coefficient records and Ws[s, t-1] blocks
  L.coef = off; off += align256((size_t)g.BH * g.nc * coef_rec_floats(pl.CH) * sizeof(float));
  L.wsh = off; off += align256((size_t)g.BH * g.nc * pl.CH * (pl.CH + kHaloPad) * pl.esize);
  // the backward's chunk records (input-only: formed in the forward's coefficient launch)
  L.bcoef = off; off += align256(brec ? (size_t)g.BH * pl.gb.nc * coef_rec_floats(pl.CHB) * sizeof(float) : 0);
  L.bwsh = off; off += align256(brec ? (size_t)g.BH * pl.gb.nc * pl.CHB * (pl.CHB + kHaloPad) * pl.esize : 0);
  L.bufc = off; off += align256(walk_with_buffer(pl) ? (size_t)g.BH * bufw::kCorrFloats * sizeof(float) : 0);
  L.total = off;
  return L;
}

// backward workspace: adjoint aggregates, segment-end adjoints, dS_ref partials, boundary partials,
// token-gate (target, lag) gradients, the scalar-gradient inputs (none for the backward of
// chunk_bwd.hip, which forms its scalar gradients in the walk).
struct BwdLayout {
  size_t agg, segadj, dsref, tail, halo, dw, scal, badj, total;
};

BwdLayout bwd_layout(const Plan& pl) {
  const Geom& g = pl.gb;
  const int nseg = pl.sgb.nseg;
  BwdLayout L{};
  const size_t st = (size_t)g.DV * g.DK * sizeof(float);
  size_t off = 0;
  L.agg = off; off += align256((size_t)g.BH * nseg * pl.sgb.agg_stride * sizeof(float));
  L.segadj = off; off += align256((size_t)g.BH * nseg * 2 * st);
  L.dsref = off; off += align256((size_t)g.BH * nseg * st);
  L.tail = off; off += align256((size_t)g.BH * nseg * g.H * (g.DV + g.DK) * sizeof(float));
  L.halo = off; off += align256((size_t)g.BH * nseg * g.H * (g.DV + g.DK) * sizeof(float));
  L.dw = off; off += align256(g.gate_mode == ATLAS_GATE_TOKEN ? (size_t)g.BH * g.T * g.e * sizeof(float) : 0);
  L.scal = off; off += align256(pl.cbwd ? 0 : (size_t)g.BH * g.nc * scalar_block_floats(pl.CHB) * sizeof(float));
  L.badj = off; off += align256(walk_with_buffer(pl) ? (size_t)g.BH * bufw::kAdjFloats * sizeof(float) : 0);
  L.total = off;
  return L;
}

// `saved` of a dual plan: the flag (256 bytes), then the segment-parallel sequence's layout, then the
// exact sequence's.
struct DualLayout {
  size_t fast, exact, total;
};
DualLayout dual_layout(const Plan& fast, const Plan& exact) {
  DualLayout D{};
  D.fast = 256;
  D.exact = D.fast + saved_layout(fast).total;
  D.total = D.exact + saved_layout(exact).total;
  return D;
}

size_t saved_bytes(const atlas_mem_problem* p, const Plan& pl) {
  if (!pl.dual) return saved_layout(pl).total;
  return dual_layout(pl, make_plan(p, true)).total;
}
size_t bwd_ws_bytes(const atlas_mem_problem* p, const Plan& pl) {
  if (!pl.dual) return bwd_layout(pl).total;
  return std::max(bwd_layout(pl).total, bwd_layout(make_plan(p, true)).total);
}

// The two sequences of a dual plan, flag-selected: the fast one always runs in the forward (and
// clears / sets the flag), the exact one only when the flag is set; the backward runs the one the
// forward's flag selected.
void set_flag(Plan& pl, const int* flag, int run, int reset, int check) {
  for (Geom* g : {&pl.g, &pl.gb}) {
    g->flag = flag; g->flag_run = run; g->flag_reset = reset; g->clamp_check = check;
  }
}

bool misaligned(const void* p, size_t a) { return p && (reinterpret_cast<uintptr_t>(p) % a) != 0; }

template <typename T>
int run_fwd(const Plan& pl, const atlas_mem_fwd_args* x, float* saved, hipStream_t s) {
  FwdPtrs<T> a;
  a.k = (const T*)x->k; a.q = (const T*)x->q; a.v = (const T*)x->v;
  a.lr = (const T*)x->lr; a.decay = (const T*)x->decay; a.beta = (const T*)x->beta; a.gate = (const T*)x->gate;
  a.S_ref = x->S_ref; a.S0 = x->S0; a.Z0 = x->Z0; a.buf_in = x->buffer_in;
  const SavedLayout SL = saved_layout(pl);
  unsigned char* sv = reinterpret_cast<unsigned char*>(saved);
  a.y = (T*)x->y; a.S_T = x->S_T; a.Z_T = x->Z_T; a.buf_out = x->buffer_out;
  a.buf_corr = nullptr;
  float* seg_states = reinterpret_cast<float*>(sv + SL.seg);
  float* agg = reinterpret_cast<float*>(sv + SL.agg);
  float* final_raw = reinterpret_cast<float*>(sv + SL.final_raw);
  float* rw = reinterpret_cast<float*>(sv + SL.rw);
  float* coef = reinterpret_cast<float*>(sv + SL.coef);
  T* wsh = reinterpret_cast<T*>(sv + SL.wsh);
  const Geom& g = pl.g;
  // chunk coefficient records of the forward and of the backward (one launch, inputs only)
  constexpr int CHF = sizeof(T) == 2 ? 64 : 32, CHB = sizeof(T) == 2 ? 32 : 16;
  hipError_t err = hipErrorInvalidValue;
  if constexpr (sizeof(T) == 2) {
    if (pl.ccoef)
      err = launch_chunk_coef_fwd(g, a.decay, a.lr, a.beta, a.gate, coef, wsh, s);
  }
  if (!pl.ccoef)
    err = launch_chunk_coef_pair<T, CHF, CHB>(
        g, pl.gb, a.decay, a.lr, a.beta, a.gate, coef, wsh, pl.cbwd ? nullptr : reinterpret_cast<float*>(sv + SL.bcoef),
        pl.cbwd ? nullptr : reinterpret_cast<T*>(sv + SL.bwsh), s);
  if (err != hipSuccess) return ATLAS_MEM_ERR_LAUNCH;
  err = hipErrorInvalidValue;
  if (g.DK == 64) {
    if constexpr (sizeof(T) == 2) {
      if (walk_fwd_supported(g)) {
        err = hipSuccess;
        if (walk_with_buffer(pl)) {
          float* corr = reinterpret_cast<float*>(sv + SL.bufc);
          err = launch_buf_state(g, a, pl.sg, coef, corr, s);
          a.buf_corr = corr;
        }
        if (err == hipSuccess) err = launch_walk_fwd(g, a, pl.sg, agg, seg_states, rw, final_raw, coef, wsh, s);
        if (err == hipSuccess && a.buf_corr) err = launch_buf_y(g, a, wsh, s);
      }
      else
        err = launch_fwd_seg<T, 64, 64>(g, a, pl.sg, agg, seg_states, rw, final_raw, coef, wsh, s);
    }
    else err = launch_fwd_seg<T, 32, 64>(g, a, pl.sg, agg, seg_states, rw, final_raw, coef, wsh, s);
  } else if (g.DK == 32) {
    if constexpr (sizeof(T) == 2) err = launch_fwd_seg<T, 64, 32>(g, a, pl.sg, agg, seg_states, rw, final_raw, coef, wsh, s);
    else err = launch_fwd_seg<T, 32, 32>(g, a, pl.sg, agg, seg_states, rw, final_raw, coef, wsh, s);
  }
  return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

template <typename T>
int run_bwd(const Plan& pl, const atlas_mem_bwd_args* x, const float* saved, void* ws, hipStream_t s) {
  const Geom& gb = pl.gb;
  const BwdLayout L = bwd_layout(pl);
  const SavedLayout SL = saved_layout(pl);
  unsigned char* w = static_cast<unsigned char*>(ws);
  const unsigned char* sv = reinterpret_cast<const unsigned char*>(saved);
  BwdPtrs<T> a{};
  a.k = (const T*)x->k; a.q = (const T*)x->q; a.v = (const T*)x->v;
  a.lr = (const T*)x->lr; a.decay = (const T*)x->decay; a.beta = (const T*)x->beta; a.gate = (const T*)x->gate;
  a.S_ref = x->S_ref; a.S0 = x->S0; a.Z0 = x->Z0; a.buf_in = x->buffer_in;
  a.dy = (const T*)x->dy; a.dS_T = x->dS_T; a.dZ_T = x->dZ_T; a.dbuf_out = x->dbuffer_out;
  a.dk = (T*)x->dk; a.dq = (T*)x->dq; a.dv = (T*)x->dv; a.dlr = (T*)x->dlr; a.ddecay = (T*)x->ddecay;
  a.dbeta = (T*)x->dbeta; a.dgate = (T*)x->dgate;
  a.dS_ref = x->dS_ref; a.dS0 = x->dS0; a.dZ0 = x->dZ0; a.dbuf_in = x->dbuffer_in;
  BwdSegPtrs p;
  p.seg_states = reinterpret_cast<const float*>(sv + SL.seg);
  p.final_raw = reinterpret_cast<const float*>(sv + SL.final_raw);
  p.adj_agg = reinterpret_cast<float*>(w + L.agg);
  p.seg_adj = reinterpret_cast<float*>(w + L.segadj);
  p.rw = reinterpret_cast<const float*>(sv + SL.rw);
  p.dsref_part = reinterpret_cast<float*>(w + L.dsref);
  p.tail_part = gb.H > 0 ? reinterpret_cast<float*>(w + L.tail) : nullptr;
  p.halo_part = gb.H > 0 ? reinterpret_cast<float*>(w + L.halo) : nullptr;
  p.dw = gb.gate_mode == ATLAS_GATE_TOKEN ? reinterpret_cast<float*>(w + L.dw) : nullptr;
  // formed by the forward (read only here)
  p.coef = const_cast<float*>(reinterpret_cast<const float*>(sv + SL.bcoef));
  p.wsh = const_cast<unsigned char*>(sv + SL.bwsh);
  p.scal = reinterpret_cast<float*>(w + L.scal);
  p.buf_adj = walk_with_buffer(pl) ? reinterpret_cast<float*>(w + L.badj) : nullptr;
  hipError_t err = hipErrorInvalidValue;
  // the specialised walks run as a pair: the forward saved its states in their layout
  const bool walk = sizeof(T) == 2 && walk_fwd_supported(pl.g);
  // the specialised path forms its adjoint aggregates over the forward's chunks and records
  const AggOverFwd agf{pl.g, pl.sg, reinterpret_cast<const float*>(sv + SL.coef), pl.cbwd};
  const bool agg_fwd = walk && pl.g.Lc == 64;
  if (gb.DK == 64) {
    if constexpr (sizeof(T) == 2) err = launch_bwd_seg<T, 32, 64>(gb, a, pl.sgb, p, s, walk, agg_fwd ? &agf : nullptr);
    else err = launch_bwd_seg<T, 16, 64>(gb, a, pl.sgb, p, s, false, nullptr);
  } else if (gb.DK == 32) {
    if constexpr (sizeof(T) == 2) err = launch_bwd_seg<T, 32, 32>(gb, a, pl.sgb, p, s, false, nullptr);
    else err = launch_bwd_seg<T, 16, 32>(gb, a, pl.sgb, p, s, false, nullptr);
  }
  return err == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

int check_bwd_args(const atlas_mem_problem& p, const atlas_mem_bwd_args* args, const float* saved,
                   const void* workspace);

// The backward of a plan (of both flag-selected sequences for a dual plan).
int run_bwd_plan(const atlas_mem_problem* prob, const Plan& pl, const atlas_mem_bwd_args* args, const float* saved,
                 void* ws, hipStream_t s) {
  auto one = [&](const Plan& q, const float* sv) {
    return prob->dtype == ATLAS_DT_BF16 ? run_bwd<bf16>(q, args, sv, ws, s) : run_bwd<float>(q, args, sv, ws, s);
  };
  if (!pl.dual) return one(pl, saved);
  Plan fast = pl, exact = make_plan(prob, true);
  const unsigned char* sv = reinterpret_cast<const unsigned char*>(saved);
  const DualLayout D = dual_layout(fast, exact);
  const int* flag = reinterpret_cast<const int*>(sv);
  set_flag(fast, flag, 0, 0, 0);
  set_flag(exact, flag, 1, 0, 0);
  // either order: the flag is only read here; the exact sequence first, so that the per-kernel
  // timing labels name the segment-parallel kernels that normally run
  const int st = one(exact, reinterpret_cast<const float*>(sv + D.exact));
  if (st != ATLAS_MEM_OK) return st;
  return one(fast, reinterpret_cast<const float*>(sv + D.fast));
}

// Scratch of atlas_mem_bwd_noalloc: the backward workspace as a file-scope device array (each GPU
// holds its own copy for the life of the process). In host code `scratch` names a host-side
// stand-in, never the device memory: its per-device address comes from hipGetSymbolAddress, looked
// up once per device with that device current (the entry point's first call there) and kept in
// scratch_dev. Calls that overlap on one GPU share the array and race; every call overwrites what
// it reads (the backward never relies on zeroed workspace), so nothing has to be cleared.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_dev[kMaxDevices] = {};

int scratch_on_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return ATLAS_MEM_ERR_LAUNCH;
  std::lock_guard<std::mutex> lk(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return ATLAS_MEM_ERR_LAUNCH;
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return ATLAS_MEM_OK;
}

}  // namespace

extern "C" {

int atlas_mem_abi_version(void) { return ATLAS_MEM_ABI_VERSION; }

const char* atlas_mem_strerror(int status) {
  switch (status) {
    case ATLAS_MEM_OK: return "ok";
    case ATLAS_MEM_ERR_ABI: return "problem.abi_version does not match the library ABI version";
    case ATLAS_MEM_ERR_SHAPE: return "unsupported sizes (need bh >= 1, seq_len >= 1, d_k == d_v in {32, 64}, 1 <= window <= 33)";
    case ATLAS_MEM_ERR_DTYPE: return "unknown dtype code (ATLAS_DT_F32 or ATLAS_DT_BF16)";
    case ATLAS_MEM_ERR_NULL: return "a required pointer is NULL";
    case ATLAS_MEM_ERR_ALIGN: return "a pointer is not aligned to its element size";
    case ATLAS_MEM_ERR_UNSUPPORTED: return "the chunk length implied by clamp_every is below 8 tokens or shorter than window - 1; split the call at clamp_every";
    case ATLAS_MEM_ERR_WORKSPACE: return "workspace smaller than atlas_mem_bwd_workspace_bytes()";
    case ATLAS_MEM_ERR_LAUNCH: return "a HIP kernel launch or runtime call failed";
    case ATLAS_MEM_ERR_ARG: return "inconsistent flags (momentum/gate/map/buffer/clamp)";
    case ATLAS_MEM_ERR_SCRATCH: return "the backward workspace exceeds the 64 MiB static scratch of atlas_mem_bwd_noalloc; use atlas_mem_bwd";
    default: return "unknown atlas_mem status";
  }
}

int atlas_mem_validate(const atlas_mem_problem* prob) { return make_plan(prob).status; }

size_t atlas_mem_saved_bytes(const atlas_mem_problem* prob) {
  const Plan pl = make_plan(prob);
  if (!pl.ok) return 0;
  return saved_bytes(prob, pl);
}

size_t atlas_mem_bwd_workspace_bytes(const atlas_mem_problem* prob) {
  const Plan pl = make_plan(prob);
  if (!pl.ok) return 0;
  return bwd_ws_bytes(prob, pl);
}

int atlas_mem_fwd(const atlas_mem_problem* prob, const atlas_mem_fwd_args* args, float* saved, void* stream) {
  const Plan pl = make_plan(prob);
  if (!pl.ok) return pl.status;
  if (!args || !saved) return ATLAS_MEM_ERR_NULL;
  const atlas_mem_problem& p = *prob;
  if (!args->k || !args->q || !args->v || !args->lr || !args->decay || !args->S_ref || !args->S0 ||
      !args->y || !args->S_T)
    return ATLAS_MEM_ERR_NULL;
  if (p.momentum && (!args->beta || !args->Z_T)) return ATLAS_MEM_ERR_NULL;
  if (!p.momentum && (args->beta || args->Z_T)) return ATLAS_MEM_ERR_ARG;
  if ((p.gate_mode != ATLAS_GATE_NONE) != (args->gate != nullptr)) return ATLAS_MEM_ERR_ARG;
  if (p.has_buffer && !args->buffer_in) return ATLAS_MEM_ERR_NULL;
  if (p.window > 1 && !args->buffer_out) return ATLAS_MEM_ERR_NULL;
  // every pointer 16-byte aligned: the kernels move rows and states with 16-byte accesses
  const void* tp[] = {args->k, args->q, args->v, args->lr, args->decay, args->beta, args->gate, args->y};
  for (const void* q : tp) if (misaligned(q, 16)) return ATLAS_MEM_ERR_ALIGN;
  const void* fp[] = {args->S_ref, args->S0, args->Z0, args->buffer_in, args->S_T, args->Z_T, args->buffer_out, saved};
  for (const void* q : fp) if (misaligned(q, 16)) return ATLAS_MEM_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto one = [&](const Plan& q, float* sv) {
    return p.dtype == ATLAS_DT_BF16 ? run_fwd<bf16>(q, args, sv, s) : run_fwd<float>(q, args, sv, s);
  };
  if (!pl.dual) return one(pl, saved);
  Plan fast = pl, exact = make_plan(prob, true);
  unsigned char* sv = reinterpret_cast<unsigned char*>(saved);
  const DualLayout D = dual_layout(fast, exact);
  const int* flag = reinterpret_cast<const int*>(sv);
  set_flag(fast, flag, -1, 1, p.clamp_every);
  set_flag(exact, flag, 1, 0, 0);
  const int st = one(fast, reinterpret_cast<float*>(sv + D.fast));
  if (st != ATLAS_MEM_OK) return st;
  return one(exact, reinterpret_cast<float*>(sv + D.exact));
}

int atlas_mem_bwd(const atlas_mem_problem* prob, const atlas_mem_bwd_args* args, const float* saved,
                  void* workspace, size_t workspace_bytes, void* stream) {
  const Plan pl = make_plan(prob);
  if (!pl.ok) return pl.status;
  if (!args || !saved || !workspace) return ATLAS_MEM_ERR_NULL;
  if (workspace_bytes < bwd_ws_bytes(prob, pl)) return ATLAS_MEM_ERR_WORKSPACE;
  const int st = check_bwd_args(*prob, args, saved, workspace);
  if (st != ATLAS_MEM_OK) return st;
  return run_bwd_plan(prob, pl, args, saved, workspace, static_cast<hipStream_t>(stream));
}

int atlas_mem_bwd_noalloc(const atlas_mem_problem* prob, const atlas_mem_bwd_args* args, const float* saved,
                          void* stream) {
  const Plan pl = make_plan(prob);
  if (!pl.ok) return pl.status;
  if (!args || !saved) return ATLAS_MEM_ERR_NULL;
  if (bwd_ws_bytes(prob, pl) > kNoAllocScratchBytes) return ATLAS_MEM_ERR_SCRATCH;
  void* ws = nullptr;
  const int ss = scratch_on_current_device(&ws);
  if (ss != ATLAS_MEM_OK) return ss;
  const int st = check_bwd_args(*prob, args, saved, ws);
  if (st != ATLAS_MEM_OK) return st;
  return run_bwd_plan(prob, pl, args, saved, ws, static_cast<hipStream_t>(stream));
}

size_t atlas_mem_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

}  // extern "C"

namespace {
// Pointer and alignment checks shared by atlas_mem_bwd and atlas_mem_bwd_noalloc (no HIP call).
int check_bwd_args(const atlas_mem_problem& p, const atlas_mem_bwd_args* args, const float* saved,
                   const void* workspace) {
  if (!args->k || !args->q || !args->v || !args->lr || !args->decay || !args->S_ref || !args->S0 ||
      !args->dk || !args->dq || !args->dv || !args->dlr || !args->ddecay || !args->dS_ref || !args->dS0)
    return ATLAS_MEM_ERR_NULL;
  if (p.momentum && (!args->beta || !args->dbeta || !args->dZ0)) return ATLAS_MEM_ERR_NULL;
  if ((p.gate_mode != ATLAS_GATE_NONE) != (args->gate != nullptr)) return ATLAS_MEM_ERR_ARG;
  if (p.gate_mode != ATLAS_GATE_NONE && !args->dgate) return ATLAS_MEM_ERR_NULL;
  if (p.has_buffer && (!args->buffer_in || !args->dbuffer_in)) return ATLAS_MEM_ERR_NULL;
  const void* tp[] = {args->k, args->q, args->v, args->lr, args->decay, args->beta, args->gate, args->dy,
                      args->dk, args->dq, args->dv, args->dlr, args->ddecay, args->dbeta, args->dgate};
  for (const void* q : tp) if (misaligned(q, 16)) return ATLAS_MEM_ERR_ALIGN;
  const void* fp[] = {args->S_ref, args->S0, args->Z0, args->buffer_in, args->dS_T, args->dZ_T, args->dbuffer_out,
                      args->dS_ref, args->dS0, args->dZ0, args->dbuffer_in, saved, workspace};
  for (const void* q : fp) if (misaligned(q, 16)) return ATLAS_MEM_ERR_ALIGN;
  return ATLAS_MEM_OK;
}
}  // namespace

extern "C" {

int atlas_mem_profile_enable(int on) {
  Profiler& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  P.on = on != 0;
  return ATLAS_MEM_OK;
}

int atlas_mem_profile_read(double* ms, long long* launches, int n, int reset) {
  Profiler& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  for (const Pending& q : P.pending) {
    float t = 0.f;
    if (hipEventSynchronize(q.b) != hipSuccess || hipEventElapsedTime(&t, q.a, q.b) != hipSuccess) return ATLAS_MEM_ERR_LAUNCH;
    P.ms[q.kid] += t;
    P.n[q.kid] += 1;
    P.pool.push_back(q.a);
    P.pool.push_back(q.b);
  }
  P.pending.clear();
  for (int i = 0; i < n && i < KID_COUNT; ++i) {
    if (ms) ms[i] = P.ms[i];
    if (launches) launches[i] = P.n[i];
  }
  if (reset) {
    for (int i = 0; i < KID_COUNT; ++i) { P.ms[i] = 0.0; P.n[i] = 0; }
  }
  return ATLAS_MEM_OK;
}

const char* atlas_mem_kernel_name(int kid) {
  return (kid >= 0 && kid < KID_COUNT) ? kKernelNames[kid] : "";
}

int atlas_mem_mfma_selftest(int dtype, const void* A, const void* B, float* C, void* stream) {
  if (!A || !B || !C) return ATLAS_MEM_ERR_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ATLAS_DT_BF16) {
    hipLaunchKernelGGL(k_mfma_selftest<bf16>, dim3(1), dim3(64), 0, s, (const bf16*)A, (const bf16*)B, C);
  } else if (dtype == ATLAS_DT_F32) {
    hipLaunchKernelGGL(k_mfma_selftest<float>, dim3(1), dim3(64), 0, s, (const float*)A, (const float*)B, C);
  } else {
    return ATLAS_MEM_ERR_DTYPE;
  }
  return hipGetLastError() == hipSuccess ? ATLAS_MEM_OK : ATLAS_MEM_ERR_LAUNCH;
}

}  // extern "C"

/*
 * atlas_mem.h - C ABI of the MI355X memory-layer recurrence library (libatlas_mem.so).
 *
 * One library, built ahead of time for gfx950, loaded with ctypes (or dlopen) by the
 * host-side mirror of the reference module API. Plain pointers and sizes only; no torch types.
 *
 * Recurrence computed per head-batch row bh (all states fp32, row-major [d_v, d_k]):
 *   phi_t = map(k_t), psi_t = map(q_t)                (map: identity or sum_{i=1..g} x^i)
 *   delta_t = S_ref phi_t - v_t
 *   g_t = sum_{j=0..e-1} w[t,j] delta_{t-j} phi_{t-j}^T   (+ carried buffer for t-j < 0)
 *   Z_t = beta_t Z_{t-1} + g_t ;  S_t = alpha_t S_{t-1} - eta_t Z_t   (no momentum: Z_t = g_t)
 *   y_t = S_{t-1} psi_t ;  S_T = clamp(S_{T-1}, -100, 100) ;  Z_T = Z_{T-1}
 * With clamp_every = n > 0, S is also clamped after every token t with (t+1) % n == 0
 * (the reference's scan_chunk_len semantics).
 *
 * Replaces the reference's native FFI:
 *   forward_exact(...)   atlas_pytorch/cuda/atlas_omega.cpp:56-99   -> atlas_mem_fwd
 *   backward_exact(...)  atlas_pytorch/cuda/atlas_omega.cpp:102-136  -> atlas_mem_bwd
 * and the AssocScan/PyTorch path it bypassed (atlas_pytorch/rnn_memory.py:605-730,
 * :300-406), whose semantics (fp32 state, buffer carry, clamp, any window e) it follows.
 *
 * Ownership: the caller allocates every buffer (outputs, the `saved` state buffer that
 * travels from forward to backward, and the backward workspace); the library never
 * allocates device memory. Calls are asynchronous on the given HIP stream (`stream` is a
 * hipStream_t passed as void*; NULL = the default stream) and stream-ordered. Entry points
 * are reentrant; concurrent calls must not share output, saved or workspace buffers.
 *
 * Errors: every entry point returns ATLAS_MEM_OK (0) or a nonzero code; the text is
 * available from atlas_mem_strerror(code). Shape/dtype/pointer checks happen before any
 * launch; a launch failure returns ATLAS_MEM_ERR_LAUNCH.
 */
#ifndef ATLAS_MEM_H
#define ATLAS_MEM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATLAS_MEM_ABI_VERSION 1

enum atlas_mem_status {
  ATLAS_MEM_OK = 0,
  ATLAS_MEM_ERR_ABI = 1,          /* problem.abi_version != ATLAS_MEM_ABI_VERSION */
  ATLAS_MEM_ERR_SHAPE = 2,        /* sizes out of the supported range */
  ATLAS_MEM_ERR_DTYPE = 3,        /* unknown dtype code */
  ATLAS_MEM_ERR_NULL = 4,         /* a required pointer is NULL */
  ATLAS_MEM_ERR_ALIGN = 5,        /* a pointer is not 16-byte aligned */
  ATLAS_MEM_ERR_UNSUPPORTED = 6,  /* valid request this build does not implement */
  ATLAS_MEM_ERR_WORKSPACE = 7,    /* workspace too small */
  ATLAS_MEM_ERR_LAUNCH = 8,       /* a HIP launch or runtime call failed */
  ATLAS_MEM_ERR_ARG = 9,          /* inconsistent flags */
  ATLAS_MEM_ERR_SCRATCH = 10      /* atlas_mem_bwd_noalloc: workspace above its static scratch */
};

enum atlas_mem_dtype { ATLAS_DT_F32 = 0, ATLAS_DT_BF16 = 1 };
enum atlas_mem_gate_mode {
  ATLAS_GATE_NONE = 0,   /* w[t,j] = 1 */
  ATLAS_GATE_TOKEN = 1,  /* gate [bh,T]: w[t,j] = u_{t-j} (reference omega_gate); buffer holds gated products */
  ATLAS_GATE_LAG = 2     /* gate [bh,T,e]: w[t,j] = U[t,j]; buffer holds ungated products */
};
enum atlas_mem_map_mode { ATLAS_MAP_OFF = 0, ATLAS_MAP_ELEMENTWISE = 1 };

typedef struct atlas_mem_problem {
  int32_t abi_version;  /* ATLAS_MEM_ABI_VERSION */
  int32_t bh;           /* batch * heads */
  int32_t seq_len;      /* T >= 1 */
  int32_t d_k;          /* key/feature width: 32, 64 */
  int32_t d_v;          /* value width (rows of S): equal to d_k in this build */
  int32_t window;       /* omega window e, 1..33 */
  int32_t momentum;     /* 1: Z recurrence with beta; 0: Z_t = g_t, no Z0/Z_T */
  int32_t gate_mode;    /* atlas_mem_gate_mode */
  int32_t map_mode;     /* atlas_mem_map_mode, applied to k and q on load */
  int32_t map_degree;   /* g for ATLAS_MAP_ELEMENTWISE (>= 1) */
  int32_t has_buffer;   /* 1: buffer_in [bh, e-1, d_v, d_k] supplied (otherwise zeros) */
  int32_t clamp_every;  /* 0 or scan_chunk_len */
  int32_t clamp_final;  /* 1: S_T = clamp(S_{T-1}) (reference PyTorch path) */
  int32_t dtype;        /* atlas_mem_dtype of k, q, v, lr, decay, beta, gate, y and their grads */
} atlas_mem_problem;

typedef struct atlas_mem_fwd_args {
  const void* k;            /* [bh, T, d_k] raw keys (feature map applied inside) */
  const void* q;            /* [bh, T, d_k] raw queries */
  const void* v;            /* [bh, T, d_v] */
  const void* lr;           /* [bh, T] eta */
  const void* decay;        /* [bh, T] alpha */
  const void* beta;         /* [bh, T] momentum; NULL iff momentum == 0 */
  const void* gate;         /* [bh, T] or [bh, T, e]; NULL iff gate_mode == NONE */
  const float* S_ref;       /* [bh, d_v, d_k] reference state for delta */
  const float* S0;          /* [bh, d_v, d_k] */
  const float* Z0;          /* [bh, d_v, d_k] or NULL (zeros); ignored without momentum */
  const float* buffer_in;   /* [bh, e-1, d_v, d_k] iff has_buffer */
  void* y;                  /* [bh, T, d_v] out */
  float* S_T;               /* [bh, d_v, d_k] out */
  float* Z_T;               /* [bh, d_v, d_k] out iff momentum, else NULL */
  float* buffer_out;        /* [bh, e-1, d_v, d_k] out iff e > 1, else NULL */
} atlas_mem_fwd_args;

typedef struct atlas_mem_bwd_args {
  /* forward inputs, the same buffers that were passed to atlas_mem_fwd */
  const void* k; const void* q; const void* v;
  const void* lr; const void* decay; const void* beta; const void* gate;
  const float* S_ref; const float* S0; const float* Z0; const float* buffer_in;
  /* incoming gradients; NULL means zero */
  const void* dy;           /* [bh, T, d_v] (dtype) */
  const float* dS_T;        /* [bh, d_v, d_k] */
  const float* dZ_T;        /* [bh, d_v, d_k] */
  const float* dbuffer_out; /* [bh, e-1, d_v, d_k] */
  /* gradients out (dtype unless noted); dbeta/dgate NULL iff the input is absent */
  void* dk; void* dq; void* dv; void* dlr; void* ddecay; void* dbeta; void* dgate;
  float* dS_ref;            /* [bh, d_v, d_k] */
  float* dS0;               /* [bh, d_v, d_k] */
  float* dZ0;               /* [bh, d_v, d_k] iff momentum, else NULL */
  float* dbuffer_in;        /* [bh, e-1, d_v, d_k] iff has_buffer, else NULL */
} atlas_mem_bwd_args;

/* Library ABI version (ATLAS_MEM_ABI_VERSION of the build). */
int atlas_mem_abi_version(void);

/* Static text for a status code. */
const char* atlas_mem_strerror(int status);

/* Checks a problem description without touching the GPU. */
int atlas_mem_validate(const atlas_mem_problem* prob);

/* Bytes of the `saved` buffer atlas_mem_fwd writes (its scratch plus the fp32 states
 * atlas_mem_bwd reuses). Returns 0 for an invalid problem. */
size_t atlas_mem_saved_bytes(const atlas_mem_problem* prob);

/* Bytes of scratch workspace atlas_mem_bwd needs. Returns 0 for an invalid problem. */
size_t atlas_mem_bwd_workspace_bytes(const atlas_mem_problem* prob);

/* Forward pass. Replaces forward_exact (atlas_pytorch/cuda/atlas_omega.cpp:56-99) and the
 * PyTorch scan path (atlas_pytorch/rnn_memory.py:605-730). `saved` (atlas_mem_saved_bytes)
 * is required; keep it unchanged until the matching atlas_mem_bwd when a backward follows. */
int atlas_mem_fwd(const atlas_mem_problem* prob, const atlas_mem_fwd_args* args,
                  float* saved, void* stream);

/* One token (seq_len == 1, forward only) without a saved buffer: the decode / streaming step of
 * RNNMemoryTransformer.generate (atlas_pytorch/rnn_transformer.py:863-900), which runs the cell's
 * recurrence (atlas_pytorch/rnn_memory.py:605-730) one token at a time. Same problem and argument
 * structures and the same results as atlas_mem_fwd at T = 1; outputs may alias their inputs
 * (S_T = S0, Z_T = Z0, buffer_out = buffer_in) for in-place state updates. One launch. */
int atlas_mem_step(const atlas_mem_problem* prob, const atlas_mem_fwd_args* args, void* stream);

/* The carried Omega buffer as rank-1 factors (the on-device RNNMemState format, dense or factored,
 * of atlas_pytorch/rnn_transformer.py:863-900's generation loop). Every dense slot the forward
 * carries is one outer product g_p delta_p phi_p^T (rnn_memory.py:673-687); the factored form holds
 *   factors [bh, e-1, d_v + d_k] fp32, slot m = (g_p delta_p [d_v] | phi_p [d_k]), slot 0 the oldest,
 * (d_v + d_k) / (d_v d_k) of the dense bytes. */

/* atlas_mem_step with the window sum over factored slots: args->buffer_in / buffer_out must be NULL;
 * factors_in (iff prob->has_buffer) -> factors_out (iff window > 1), which must not overlap
 * (callers alternate two buffers). S_T = S0 and Z_T = Z0 may alias as in atlas_mem_step. */
int atlas_mem_step_factored(const atlas_mem_problem* prob, const atlas_mem_fwd_args* args, const float* factors_in,
                            float* factors_out, void* stream);

/* The factors the buffer holds after prob->seq_len tokens: the last e-1 of [factors_in; tokens],
 * i.e. the factored form of atlas_mem_fwd's buffer_out (k [bh, T, d_k], v [bh, T, d_v], gate as
 * in atlas_mem_fwd_args, S_ref [bh, d_v, d_k]); window >= 2; factors_in iff has_buffer, not
 * overlapping factors_out. */
int atlas_buffer_factors(const atlas_mem_problem* prob, const void* k, const void* v, const void* gate,
                         const float* S_ref, const float* factors_in, float* factors_out, void* stream);

/* factors [bh, slots, d_v + d_k] -> dense [bh, slots, d_v, d_k] (the buffer_in of atlas_mem_fwd and
 * RNNMemState.omega_buffer). */
int atlas_buffer_expand(int bh, int slots, int d_v, int d_k, const float* factors, float* dense, void* stream);

/* Backward pass from the forward's `saved` states. Replaces backward_exact
 * (atlas_pytorch/cuda/atlas_omega.cpp:102-136) plus the PyTorch-side chain in
 * AtlasOmegaFunction.backward (atlas_pytorch/cuda/atlas_omega_autograd.py:156-204). */
int atlas_mem_bwd(const atlas_mem_problem* prob, const atlas_mem_bwd_args* args,
                  const float* saved, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free backward. No counterpart in the reference: for callers that cannot allocate
 * device memory (code under HIP graph capture, tight training loops, harnesses that forbid
 * hipMalloc). Same problem, arguments, kernels and results as atlas_mem_bwd, with the workspace
 * taken from a static device array of atlas_mem_noalloc_scratch_bytes() (64 MiB) that each GPU
 * holds for the life of the process; the library allocates nothing. Problems whose
 * atlas_mem_bwd_workspace_bytes exceeds it return ATLAS_MEM_ERR_SCRATCH (the C2, C3 and C5
 * headline shapes need 38-58 MiB). The first call on a device looks the array up with that device
 * current (make a first call outside graph capture). Calls that overlap on one GPU share the array
 * and race: serialise them (one stream, or events). */
int atlas_mem_bwd_noalloc(const atlas_mem_problem* prob, const atlas_mem_bwd_args* args,
                          const float* saved, void* stream);

/* Size of the static scratch array of atlas_mem_bwd_noalloc, in bytes. */
size_t atlas_mem_noalloc_scratch_bytes(void);

/* ---- scan primitives (row-major [n, t, d] buffers of `dtype`, gates [n, t]) -------------- */

/* out_t = gates_t * out_{t-1} + x_t, out_{-1} = prev ([n, d]) or 0 when prev is NULL.
 * Replaces assoc_scan.AssocScan.__call__(gates, inputs, prev) as called at
 * atlas_pytorch/rnn_memory.py:363,369,698,700,705 and atlas_pytorch/omega.py:267,315
 * (the T-output form; the caller prepends prev for remove_prev=False). */
int atlas_scan_fwd(int dtype, int64_t n, int64_t t, int64_t d, const void* gates, const void* x,
                   const void* prev, void* out, void* stream);

/* Gradients of atlas_scan_fwd given its output `out`: dx [n,t,d], dgates [n,t], dprev [n,d]
 * (dprev may be NULL). */
int atlas_scan_bwd(int dtype, int64_t n, int64_t t, int64_t d, const void* gates, const void* out,
                   const void* prev, const void* dout, void* dx, void* dgates, void* dprev, void* stream);

/* Inclusive window sum along t: reverse == 0: y_t = sum_{k=max(0,t-w+1)}^{t} x_k;
 * reverse == 1: y_t = sum_{k=t}^{min(t+w-1,T-1)} x_k (the adjoint). Replaces
 * _sliding_sum_along_time (atlas_pytorch/rnn_memory.py:50-61) and _sliding_sum_along_n
 * (atlas_pytorch/omega.py:24-33). */
int atlas_window_sum(int dtype, int64_t n, int64_t t, int64_t d, int window, int reverse,
                     const void* x, void* y, void* stream);

/* Right-affine scan H_t = H_{t-1} A_t + B_t over t = 1..T, fp32 (replaces affine_associative_scan,
 * atlas_pytorch/affine_scan.py:36-158): A [n,t,d,d], B [n,t,r,d], prev = H_0 [n,r,d] (NULL: zero),
 * out = H_1..H_T [n,t,r,d]; r, d <= 64. Chunked on the fp32 matrix cores: the chunks' composed maps,
 * a chain over chunks, then every chunk's states. `workspace` (atlas_affine_scan_workspace_bytes) is
 * caller-owned scratch; pointers 4-byte aligned. */
int atlas_affine_scan_fwd(int n, int t, int r, int d, const float* A, const float* B, const float* prev,
                          float* out, void* workspace, size_t workspace_bytes, void* stream);

/* Gradients of atlas_affine_scan_fwd given its output H (= out): dA [n,t,d,d], dB [n,t,r,d] and
 * dprev [n,r,d] (may be NULL) for the output gradient dout [n,t,r,d]. The adjoint is the same chunked
 * scan run backwards over A^T; same workspace size as the forward. */
int atlas_affine_scan_bwd(int n, int t, int r, int d, const float* A, const float* H, const float* prev,
                          const float* dout, float* dA, float* dB, float* dprev, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Bytes of workspace the affine scan (either direction) needs; 0 for invalid sizes. */
size_t atlas_affine_scan_workspace_bytes(int n, int t, int r, int d);

/* Tensor polynomial feature map, fused (replaces the 'tensor' mode of PolynomialFeatureMap,
 * atlas_pytorch/rnn_memory.py:125-130, which materialises vec(x x^T) with einsum / cat / matmul):
 *   pre = [x; vec(x x^T)] P,  out = sum_{i=1..degree} pre^i  (degree 1: out = pre),
 *   x [n, d_in], P [d_in + d_in^2, d_out] (row d_in + a*d_in + b multiplies x_a x_b),
 *   out, pre [n, d_out] (pre written only for degree > 1, for the backward), all of one dtype:
 *   ATLAS_DT_BF16 (bf16 matrix cores, fp32 accumulation) or ATLAS_DT_F32 (fp32 operands on the fp32
 *   matrix cores, as the reference runs the map in x.dtype).
 * degree > 1 is the elementwise map after the projection (BASELINE config C4's composition).
 * The forward takes P transposed (proj_t [d_out, d_in + d_in^2]); d_in in {16, 32, 64}, d_out a
 * multiple of 16 up to 128 (bf16 at d_in {32, 64} x d_out {32, 64, 128} runs the fast kernels),
 * degree 1..16; every pointer 16-byte aligned. */
int atlas_tensor_map_fwd(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x, const void* proj_t,
                         void* out, void* pre, void* stream);

/* Gradient of atlas_tensor_map_fwd with respect to x for the output gradient dout [n, d_out]
 * (P is a fixed buffer in the reference: no gradient). Takes P itself (proj [d_in + d_in^2, d_out])
 * and, for degree > 1, the forward's pre; dx [n, d_in] in the same dtype. */
int atlas_tensor_map_bwd(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x, const void* proj,
                         const void* pre, const void* dout, void* dx, void* stream);

/* The projection of the symmetric x x^T needs only its upper triangle: proj_sym [d_in + d_in^2, d_out]
 * holds P's linear rows and, for the quadratic rows a*d_in + b, P[a][b] + P[b][a] (b > a), P[a][a]
 * (b = a), 0 (b < a), so that [x; vec(x x^T)] proj_sym = [x; vec(x x^T)] P; proj_sym_t is its
 * transpose [d_out, d_in + d_in^2]. Same dtype, sizes and alignment as atlas_tensor_map_fwd.
 * Internal to this library (no counterpart in the reference: a preparation step of the two calls
 * below, in place of the forward's transposition of P). */
int atlas_tensor_map_symmetrize(int dtype, int d_in, int d_out, const void* proj, void* proj_sym, void* proj_sym_t,
                                void* stream);

/* atlas_tensor_map_fwd on a table from atlas_tensor_map_symmetrize (proj_sym_t in place of proj_t;
 * any other table gives wrong results): the bf16 d_in = 64 kernels skip the products over its zero
 * lower triangle (a quarter of the quadratic block's matrix-core work). The backward takes either
 * table (atlas_tensor_map_bwd with proj_sym gives the same dx). */
int atlas_tensor_map_fwd_sym(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x,
                             const void* proj_sym_t, void* out, void* pre, void* stream);

/* atlas_tensor_map_bwd on the symmetrised table proj_sym [d_in + d_in^2][d_out] (internal, no
 * reference counterpart; requires the table of atlas_tensor_map_symmetrize, any other table gives
 * wrong results): the bf16 d_in = 64 kernel halves the matrix-core work of the blocks of rows
 * a >= d_in / 2. Same arguments and results as atlas_tensor_map_bwd given proj_sym. */
int atlas_tensor_map_bwd_sym(int dtype, int64_t n, int d_in, int d_out, int degree, const void* x,
                             const void* proj_sym, const void* pre, const void* dout, void* dx, void* stream);

/* ---- state blocks for head sizes above 64 (BASELINE C4: d_k = 128, d_v = 64) ----------------
 * The recurrence with S [d_v, d_k] runs as 64 x 64 blocks S[i, j] stacked along the row axis
 * (r = (i * d_k/64 + j) * bh + b), each with S_ref = 0 and v = -delta[rows of block i], where
 * delta = S_ref phi - v couples the column blocks (replaces the full-state einsum of
 * atlas_pytorch/rnn_memory.py:659-660 for such sizes). d_k, d_v multiples of 64, <= 256. */

/* phi, psi [bh, T, d_k], v [bh, T, d_v], S_ref [bh, d_v, d_k] fp32 -> phi_b, psi_b, nv_b [NB bh, T, 64]
 * (NB = d_v/64 * d_k/64): the column blocks of phi and psi and the row blocks of v - S_ref phi. */
int atlas_block_split(int dtype, int bh, int seq_len, int d_k, int d_v, const void* phi, const void* psi, const void* v,
                      const float* S_ref, void* phi_b, void* psi_b, void* nv_b, void* stream);

/* Adjoint of atlas_block_split: dphi_b, dpsi_b, dnv_b -> dphi, dpsi [bh, T, d_k], dv [bh, T, d_v] and
 * dsref_part [bh][atlas_block_parts(T)][d_v][d_k] fp32 (sum over the second axis: dS_ref). */
int atlas_block_merge(int dtype, int bh, int seq_len, int d_k, int d_v, const void* phi, const float* S_ref,
                      const void* dphi_b, const void* dpsi_b, const void* dnv_b, void* dphi, void* dpsi, void* dv,
                      float* dsref_part, void* stream);

/* Number of dS_ref partials atlas_block_merge writes per row for seq_len tokens. */
int atlas_block_parts(int seq_len);

/* The per-token scalars (lr, decay, beta, gate) shared by every block, copied along the stacked row
 * axis, and the adjoint (replaces the expand / reshape copies and their gradient sums of the block
 * stacking, and the sum of y over the column blocks). For each of count <= 4 arrays of n[z]
 * elements of dtype:
 *   ATLAS_REPLICATE:   dst[z][r n + i] = src[z][i],                 r < nrep
 *   ATLAS_REPLICA_SUM: dst[z][i] = sum_{r < nrep} src[z][r n + i]   (fp32, in order r = 0, 1, ...)
 * nrep <= 64. Arrays with n % 8 == 0 and 16-byte aligned pointers move in 16-byte accesses. */
enum { ATLAS_REPLICATE = 0, ATLAS_REPLICA_SUM = 1 };
int atlas_replicas(int op, int dtype, int count, int nrep, const int64_t* n, const void* const* src,
                   void* const* dst, void* stream);

/* ---- cell prologue (atlas_pytorch/rnn_memory.py:567-653, MultiheadRMSNorm :139-147) --------
 * Fused around the cell's projections, which stay plain GEMMs (hipBLASLt): dtype is ATLAS_DT_F32 or
 * ATLAS_DT_BF16 for every tensor argument except inv_rms and the *_part partial sums (fp32).
 * Parameter gradients come back as per-workgroup partials [atlas_prologue_num_workgroups, ...] that
 * the caller sums over their first axis. */

/* Workgroups of atlas_prologue_* / atlas_heads_* for (batch, seq_len): the first axis of every
 * *_part buffer. */
int atlas_prologue_num_workgroups(int batch, int seq_len);

/* Sums over rows of fp32 partials (the *_part buffers of the kernels below), up to eight arrays in
 * one launch: outs[z] [cols[z]] = sum_r parts[z][r][:] in out_dtypes[z] (ATLAS_DT_BF16 or
 * ATLAS_DT_F32), summed in a fixed order (deterministic). parts, outs, cols and out_dtypes are host
 * arrays of count entries; rows = 0 writes zeros. */
int atlas_partials_sum(int count, int rows, const int* cols, const float* const* parts, void* const* outs,
                       const int* out_dtypes, void* stream);

/* xn = RMSNorm(x) = x rsqrt(mean_c x^2 + eps) norm_w (nn.RMSNorm(dim), the cell's pre_norm) and, when
 * conv_k > 1, the three depthwise convolutions over time of xn (Conv1d(dim, dim, conv_k, padding =
 * conv_k / 2, groups = dim, bias = False) truncated to seq_len: q_in[t] = sum_j wq[c][j] xn[t + j - conv_k/2]).
 * x, xn, q_in, k_in, v_in [batch, seq_len, dim]; norm_w [dim]; wq, wk, wv [dim][conv_k] (the conv
 * weights [dim, 1, conv_k]); inv_rms [batch, seq_len] fp32 out (kept for the backward). conv_k <= 8;
 * conv_k <= 1: no convolution (wq .. v_in unused). */
int atlas_prologue_fwd(int dtype, int batch, int seq_len, int dim, int conv_k, float eps, const void* x,
                       const void* norm_w, const void* wq, const void* wk, const void* wv, void* xn, void* q_in,
                       void* k_in, void* v_in, float* inv_rms, void* stream);

/* Adjoint of atlas_prologue_fwd: dxn (the gradient reaching xn directly) and dq_in / dk_in / dv_in
 * -> dx, dnorm_w_part [nwg][dim] and dconv_part [nwg][3][dim][conv_k] (q, k, v taps). */
int atlas_prologue_bwd(int dtype, int batch, int seq_len, int dim, int conv_k, const void* x, const void* norm_w,
                       const void* wq, const void* wk, const void* wv, const float* inv_rms, const void* dxn,
                       const void* dq_in, const void* dk_in, const void* dv_in, void* dx, float* dnorm_w_part,
                       float* dconv_part, void* stream);

/* The head split of the projections ql, kl, vl [batch, seq_len, heads * d] into [(batch heads), seq_len, d],
 * MultiheadRMSNorm of q and k (x / max(|x| d^-1/2, 1e-8) * gamma[h]; q_gamma, k_gamma [heads][d], both
 * NULL: no norm), and n_gates sigmoid gate heads from the logits zl [batch, seq_len, n_gates * heads]
 * plus gate_bias [n_gates * heads] into gates [n_gates][(batch heads), seq_len]. d a multiple of 8 up to
 * 128, batch * heads <= 65535, n_gates <= 8; the row tensors and gammas 16-byte aligned. */
int atlas_heads_fwd(int dtype, int batch, int seq_len, int heads, int d, int n_gates, const void* ql, const void* kl,
                    const void* vl, const void* zl, const void* q_gamma, const void* k_gamma, const void* gate_bias,
                    void* q, void* k, void* v, void* gates, void* stream);

/* Adjoint of atlas_heads_fwd given its gates: dq, dk, dv [(batch heads), seq_len, d], dgates
 * [n_gates][(batch heads), seq_len] (NULL: zero) -> dql, dkl, dvl [batch, seq_len, heads * d],
 * dzl [batch, seq_len, n_gates * heads], dq_gamma_part, dk_gamma_part [nwg][heads][d], dbias_part
 * [nwg][n_gates * heads] with nwg = atlas_prologue_num_workgroups(batch, seq_len) (every entry written;
 * the gradients are the sums over nwg). */
int atlas_heads_bwd(int dtype, int batch, int seq_len, int heads, int d, int n_gates, const void* ql, const void* kl,
                    const void* q_gamma, const void* k_gamma, const void* gates, const void* dq, const void* dk,
                    const void* dv, const void* dgates, void* dql, void* dkl, void* dvl, void* dzl,
                    float* dq_gamma_part, float* dk_gamma_part, float* dbias_part, void* stream);

/* The linear layers' products in bf16 (fp32 accumulation), up to four independent problems per
 * launch sharing m: for problem z, with A [m][k[z]] row-major,
 *   ATLAS_GEMM_NT:  C [m][n[z]] = A B^T, B [n[z]][k[z]]   (y = x W^T, the layer's forward)
 *   ATLAS_GEMM_NN:  C [m][n[z]] = A B,   B [k[z]][n[z]]   (dx = dy W, its input gradient)
 * Replaces the products autograd forms for the cell's LinearNoBias to_q / to_k / to_v / to_out and
 * its gate heads (rnn_memory.py:486-489, :503-520); the prologue's four projections and their four
 * input gradients are one launch each. n, k multiples of 8; every pointer 16-byte aligned; a, b, c
 * are host arrays of count device pointers. */
enum atlas_gemm_layout { ATLAS_GEMM_NT = 0, ATLAS_GEMM_NN = 1 };
int atlas_linear_batch(int b_layout, int count, int64_t m, const int* n, const int* k, const void* const* a,
                       const void* const* b, void* const* c, void* stream);

/* Weight gradient of a bias-free linear layer y = x W^T over n tokens: dW [out_features][in_features]
 * = sum_t dy[t]^T x[t], from dy [n][out_features] and x [n][in_features] as stored (bf16, row-major,
 * 16-byte aligned). Replaces the weight gradient autograd forms for the cell's projections
 * (nn.Linear / LinearNoBias to_q, to_k, to_v, to_out and the gate heads, rnn_memory.py:486-489,
 * :503-520). Feature counts multiples of 8; fp32 accumulation; dW in out_dtype (ATLAS_DT_BF16 or
 * ATLAS_DT_F32). The token axis is split over workgroups whose fp32 partial tiles go to workspace
 * (at least atlas_linear_wgrad_workspace_bytes) and are summed in a fixed order (deterministic).
 * n = 0 writes zeros (dy, x and workspace may then be NULL). */
int64_t atlas_linear_wgrad_workspace_bytes(int64_t n, int out_features, int in_features);
int atlas_linear_wgrad(int out_dtype, int64_t n, int out_features, int in_features, const void* dy, const void* x,
                       void* dw, void* workspace, int64_t workspace_bytes, void* stream);

/* The same for up to four layers over the same n tokens in one launch (the prologue's q / k / v /
 * gate weights): out_features, in_features, dy, x and dw are host arrays of count entries, the
 * workspace (atlas_linear_wgrad_batch_workspace_bytes, -1 for invalid sizes) holds every layer's
 * partials. */
int64_t atlas_linear_wgrad_batch_workspace_bytes(int count, int64_t n, const int* out_features,
                                                 const int* in_features);
int atlas_linear_wgrad_batch(int out_dtype, int count, int64_t n, const int* out_features, const int* in_features,
                             const void* const* dy, const void* const* x, void* const* dw, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* ---- diagnostics (no reference counterpart) ------------------------------------------------ */

/* Number of kernels the timing hooks distinguish (index -> atlas_mem_kernel_name). */
#define ATLAS_MEM_NKERNELS 14

/* Opt-in timing: while enabled, each kernel launch of atlas_mem_fwd/atlas_mem_bwd is bracketed
 * by HIP events on its stream (adds two event records per launch). */
int atlas_mem_profile_enable(int on);

/* Waits for the recorded events and returns accumulated milliseconds and launch counts per kernel
 * (arrays of n <= ATLAS_MEM_NKERNELS entries; either may be NULL); reset != 0 clears the totals. */
int atlas_mem_profile_read(double* ms, long long* launches, int n, int reset);

/* Kernel name for a timing index ("" if out of range). */
const char* atlas_mem_kernel_name(int kid);

/* Diagnostic: C[16,16] = A[16,64] * B[16,64]^T through the library's MFMA tile helpers
 * (dtype selects bf16 or fp32 inputs; C is fp32). No reference counterpart; used by the
 * GPU tests to check the matrix-core lane layout in isolation. */
int atlas_mem_mfma_selftest(int dtype, const void* A, const void* B, float* C, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_MEM_H */

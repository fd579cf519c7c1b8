/*
 * nsq_hip.h - C ABI of the MI355X (gfx950) Hyena long-convolution library.
 *
 * Plain C: pointers, sizes and an opaque stream handle (a hipStream_t passed as
 * void*; NULL = the default stream).  Every call is asynchronous on that stream,
 * performs no host synchronisation and no device allocation: the caller owns
 * every input, output and workspace buffer (size the workspace with the
 * matching *_workspace_bytes call).  The library owns only an immutable
 * per-device twiddle table built by nsq_init() or lazily on first use.
 *
 * Status: 0 (NSQ_OK) on success, otherwise an NSQ_ERR_* code with a message
 * available from nsq_last_error() (thread-local).
 *
 * Tensor layouts are row-major and contiguous:
 *   x, y, g, gx : [B, H, L]  in `dtype` (NSQ_DTYPE_*)
 *   k, gk       : [H, K]     float32 (a shared filter; the Python layer
 *                            squeezes the reference's [1, H, K])
 *   shortcut    : [H]        in `dtype` (may be NULL: no shortcut term)
 *   gs          : [H]        float32 (may be NULL when shortcut is NULL)
 */
#ifndef NSQ_HIP_H_
#define NSQ_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSQ_ABI_VERSION 16

enum {
  NSQ_OK = 0,
  NSQ_ERR_INVALID_ARGUMENT = 1,
  NSQ_ERR_UNSUPPORTED = 2,
  NSQ_ERR_HIP = 3
};

enum { NSQ_DTYPE_F32 = 0, NSQ_DTYPE_BF16 = 1, NSQ_DTYPE_F16 = 2 };

enum { NSQ_DIR_FWD = 0, NSQ_DIR_BWD = 1 };

/* Library version of this ABI (NSQ_ABI_VERSION). */
int nsq_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* nsq_last_error(void);

/* Builds the twiddle table for the current device (optional: done lazily). */
int nsq_init(void);

/*
 * 1D causal FFT convolution (+ per-channel shortcut), fused
 *   pad -> real FFT -> x filter spectrum -> inverse FFT -> crop -> cast -> + s*x.
 *
 * Replaces the native kernel the reference binds at
 *   nvsubquadratic/ops/fftconv_custom.py:286-304  (_subq_causal_conv1d_bhl ->
 *   subquadratic_ops_torch.fft_causal_conv1d(x, w)) together with the shortcut
 *   epilogue of causal_fftconv1d_bhl, fftconv_custom.py:307-335.
 * Results follow the reference torch.fft path
 *   nvsubquadratic/ops/fftconv.py:546-600 (causal_fftconv1d_fp32_bhl):
 *   y[b,h,n] = sum_m k[h,m] x[b,h,n-m] over the FFT length min(L+K, 2L), i.e.
 *   including the circular wrap-around that length implies when K > L+1.
 * Requires 1 <= K <= 2L.
 *
 * Workspace: FFT lengths above 16384 use a workspace of complex64 rows.
 * nsq_fftconv1d_causal_workspace_bytes(.., NSQ_DIR_FWD) is the minimum for the
 * forward; (.., NSQ_DIR_BWD) is the size the backward needs.  A forward given a
 * workspace of at least the NSQ_DIR_BWD size keeps its transformed x and k in
 * it ("forward state"), and a backward called with fwd_state = 1 on that same,
 * untouched workspace (same x, k) reuses them instead of transforming x and k
 * again.  The backward consumes the state: call it once per forward.
 * Shorter FFT lengths need no workspace (0 bytes; the pointer may be NULL).
 */
size_t nsq_fftconv1d_causal_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int direction);

int nsq_fftconv1d_causal_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype,
                             int64_t B, int64_t H, int64_t L, int64_t K, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Backward of nsq_fftconv1d_causal_fwd given the upstream gradient g:
 *   gx = cast(corr(g, k)) + s*g,  gk[h] = sum_b corr(g_b, x_b)[0:K] (fp32),
 *   gs[h] = sum_{b,n} g*x (fp32).
 * This is the adjoint autograd derives for the reference path
 *   (nvsubquadratic/ops/fftconv.py:583-599; the external kernel's autograd
 *   exercised by tests/ops/test_fftconv_custom_1d.py:183-200).
 */
int nsq_fftconv1d_causal_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                             float* gk, float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K,
                             void* workspace, size_t workspace_bytes, int fwd_state, void* stream);

/*
 * Per-sample (FiLM) filters for the causal 1D FFT convolution: the calls above
 * with a kernel batch.  k, gk: [kbatch*H, K] float32, kbatch = 1 (identical to
 * nsq_fftconv1d_causal_*) or B (image b convolved with filter row b*H + h);
 * gs: [kbatch*H] float32 partials (the caller sums over kbatch).  Workspace and
 * fwd_state as above, sized by nsq_fftconv1d_causal_film_workspace_bytes.
 * The reference's native wrapper rejects these filters
 * (nvsubquadratic/ops/fftconv_custom.py:294-300); its torch path accepts them
 * (nvsubquadratic/ops/fftconv.py:546-600, kernel [1|B, H, K]), and these calls
 * follow that path.
 */
size_t nsq_fftconv1d_causal_film_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                                                 int direction);

int nsq_fftconv1d_causal_film_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                                  int64_t H, int64_t L, int64_t K, int64_t kbatch, void* workspace,
                                  size_t workspace_bytes, void* stream);

int nsq_fftconv1d_causal_film_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                                  float* gk, float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K,
                                  int64_t kbatch, void* workspace, size_t workspace_bytes, int fwd_state,
                                  void* stream);

/*
 * 1D circular (periodic) FFT convolution (+ shortcut), FFT length L (no padding):
 *   y[b,h,n] = sum_{j<K} k[b|0,h,j] x[b,h,(n + (K-1)//2 - j) mod L],
 *   y = y.to(dtype) + shortcut * x.
 * k: [kbatch*H, K] float32, kbatch = 1 (shared) or B (per-sample FiLM kernels);
 * gk likewise; gs: [kbatch*H] float32 partials (the caller sums over kbatch).
 * 1 <= K <= L; L must be a power of two <= 16384 (NSQ_ERR_UNSUPPORTED
 * otherwise; L < 16 runs on its periodic extension at length 16).  No workspace.  Replaces nvsubquadratic/ops/circular_fftconv.py:310-404
 * (circular_fftconv1d_fp32_bhl, torch.fft in the reference; its autograd for the
 * backward): gx = corr(g, k) + s*g, gk[j] = sum_{b,n} g[n] x[(n + (K-1)//2 - j) mod L],
 * gs = sum g*x.
 */
int nsq_circular_fftconv1d_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                               int64_t H, int64_t L, int64_t K, int64_t kbatch, void* stream);

int nsq_circular_fftconv1d_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                               float* gk, float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K,
                               int64_t kbatch, void* stream);

/*
 * Non-causal 1D FFT convolution with a per-axis boundary (periodic bit 0):
 *   periodic = 0: zero-padded "same" conv, replaces the reference's
 *     fftconv1d_fp32_bhl (nvsubquadratic/ops/fftconv.py:603-660) and
 *     mixed_fftconv1d_fp32_bhl with periodic=(False,) (ops/mixed_fftconv.py:504-630,
 *     recipe :295-342):  y[n] = sum_j k[j] x[n + K/2 - j], x zero outside
 *     [0, L), n in [0, L); K <= 2L; L + ceil(K/2) <= 2^24, else
 *     NSQ_ERR_UNSUPPORTED.
 *   periodic = 1: the circular conv of nsq_circular_fftconv1d_fwd, for power-of-
 *     two L <= 2^24.
 * Then y is rounded to the I/O dtype and shortcut * x added (as the causal op).
 * kbatch 1 or B.  FFT lengths <= 16384 run the fused kernels and need no
 * workspace; longer ones the 4-step plan, with a workspace of
 * nsq_mixed_fftconv1d_workspace_bytes (NSQ_DIR_FWD / NSQ_DIR_BWD).  The
 * backward writes gx, gk ([kbatch*H, K]) and, with a shortcut, gs ([kbatch*H]
 * partial sums).
 */
size_t nsq_mixed_fftconv1d_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                                           unsigned periodic, int dtype, int direction);

int nsq_mixed_fftconv1d_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                            int64_t H, int64_t L, int64_t K, int64_t kbatch, unsigned periodic, void* workspace,
                            size_t workspace_bytes, void* stream);

int nsq_mixed_fftconv1d_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk,
                            float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                            unsigned periodic, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Hyena-gated causal 1D FFT convolution: the long conv
 * with the gates around it fused into its first and last passes,
 *   z = q * act1(k_gate);  y1 = causal_conv(z; k) + shortcut * z;  y = y1 * act2(v),
 * as nvsubquadratic/modules/hyena_nd.py:546 (first gate), :558 (CKConvND global
 * conv with its shortcut, ckconv_nd.py:1054-1062) and :570 (second gate) compute
 * it; each elementwise product rounded to `dtype` as those torch ops round.
 * act codes: NSQ_GATE_IDENTITY, NSQ_GATE_SIGMOID, NSQ_GATE_SILU (torch.nn.Identity,
 * Sigmoid, SiLU).  q, k_gate, v, y, y1, g, dq, dk_gate, dv: [B, H, L] in `dtype`;
 * k, gk, gs, kbatch as nsq_fftconv1d_causal_film_*.  The forward writes y1 when
 * y1 != NULL (the backward needs it).  The backward returns dq, dk_gate, dv, gk, gs.
 * Forward: FFT lengths <= 16384 run one fused kernel (no workspace); longer ones
 * run elementwise gate kernels around the multi-kernel conv.  Backward: the
 * elementwise gate kernels around the plain conv adjoint (a one-kernel gated
 * adjoint carries five extra operand streams through a latency-bound kernel and
 * measured slower on MI355X, so it is not built); fuse_gates is reserved and must
 * be 0.  Workspace: nsq_gated_fftconv1d_causal_workspace_bytes; the backward and
 * the multi-kernel forward need 16-byte aligned tensors.
 * No counterpart in the reference: there the gates are separate torch ops
 * around fft_causal_conv1d.
 */
enum { NSQ_GATE_IDENTITY = 0, NSQ_GATE_SIGMOID = 1, NSQ_GATE_SILU = 2 };

size_t nsq_gated_fftconv1d_causal_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                                                  int dtype, int direction);

int nsq_gated_fftconv1d_causal_fwd(const void* q, const void* k_gate, const void* v, const float* k,
                                   const void* shortcut, void* y, void* y1, int dtype, int act1, int act2, int64_t B,
                                   int64_t H, int64_t L, int64_t K, int64_t kbatch, void* workspace,
                                   size_t workspace_bytes, void* stream);

int nsq_gated_fftconv1d_causal_bwd(const void* g, const void* q, const void* k_gate, const void* v, const void* y1,
                                   const float* k, const void* shortcut, void* dq, void* dk_gate, void* dv, float* gk,
                                   float* gs, int dtype, int act1, int act2, int64_t B, int64_t H, int64_t L,
                                   int64_t K, int64_t kbatch, int fuse_gates, void* workspace, size_t workspace_bytes,
                                   void* stream);

/*
 * Hyena-gated 2D/3D FFT convolution (the N-d layers,
 * nvsubquadratic/modules/hyena_nd.py:546-570 around the CKConvND global conv,
 * ckconv_nd.py:1054-1062): z = q act1(k_gate), y1 = conv_nd(z) + shortcut z,
 * y = y1 act2(v), with the N-d conv of nsq_mixed_fftconv_nd_fwd (periodic mask,
 * 0 = zero-padded "same" on every axis).  The gates run as elementwise kernels
 * around the conv; each product is rounded to the I/O dtype.  y1 (may be null)
 * keeps the pre-gate output for the backward.  Tensors are 16-byte aligned.
 * The backward recomputes z and writes dq, dk_gate, dv (I/O dtype), gk
 * [kbatch*H, prod K] and, with a shortcut, gs [kbatch*H] partials.
 */
size_t nsq_gated_fftconv_nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                                            int64_t kbatch, unsigned periodic, int dtype, int direction);

int nsq_gated_fftconv_nd_fwd(int nd, const void* q, const void* k_gate, const void* v, const float* k,
                             const void* shortcut, void* y, void* y1, int dtype, int act1, int act2, int64_t B,
                             int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch, unsigned periodic,
                             void* workspace, size_t workspace_bytes, void* stream);

int nsq_gated_fftconv_nd_bwd(int nd, const void* g, const void* q, const void* k_gate, const void* v, const void* y1,
                             const float* k, const void* shortcut, void* dq, void* dk_gate, void* dv, float* gk,
                             float* gs, int dtype, int act1, int act2, int64_t B, int64_t H, const int64_t* S,
                             const int64_t* K, int64_t kbatch, unsigned periodic, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Depthwise causal direct convolution, nn.Conv1d tap order with left padding
 * K-1 (tests/ops/test_causal_conv1d_custom.py:65-72):
 *   y[b,c,n] = act( sum_{j<K} w[c,j] x[b,c,n-K+1+j] + bias[c] ),  1 <= K <= 256,
 *   act = identity (activation 0) or silu (activation 1).
 * x, y, gy, gx: [B, C, L] in `dtype`; weight, gweight: [C, K] float32;
 * bias, gbias: [C] float32 (may be NULL; gbias NULL skips its gradient).
 * Replaces subquadratic_ops_torch.causal_conv1d bound at
 *   nvsubquadratic/ops/causal_conv1d_custom.py:81-98 (its autograd backward
 *   included), used by nvsubquadratic/modules/subq_ops_causal_conv1d.py:77-83.
 */
enum { NSQ_ACT_IDENTITY = 0, NSQ_ACT_SILU = 1 };

int nsq_causal_conv1d_fwd(const void* x, const float* weight, const float* bias, void* y, int dtype, int activation,
                          int64_t B, int64_t C, int64_t L, int64_t K, void* stream);

size_t nsq_causal_conv1d_bwd_workspace_bytes(int64_t B, int64_t C, int64_t L, int64_t K, int activation);

int nsq_causal_conv1d_bwd(const void* gy, const void* x, const float* weight, const float* bias, void* gx,
                          float* gweight, float* gbias, int dtype, int activation, int64_t B, int64_t C, int64_t L,
                          int64_t K, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free variant of nsq_causal_conv1d_bwd: the same kernels and the
 * same results (bitwise), with the scratch they need (the weight / bias
 * gradient partials, and above 16 taps with silu the pre-activation gradient)
 * in a fixed device buffer of NSQ_NOALLOC_SCRATCH_BYTES that the library holds
 * on each GPU it runs on until the process ends, instead of a caller
 * workspace.  It has no counterpart in the reference: it is for callers that
 * cannot allocate device memory, such as code under HIP graph capture or a
 * serving loop that forbids allocation.  It calls no hipMalloc / hipFree.
 * Shapes whose scratch (nsq_causal_conv1d_bwd_workspace_bytes) exceeds the
 * buffer return NSQ_ERR_UNSUPPORTED without launching anything.  Every call
 * on one GPU shares that GPU's buffer: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.
 */
#define NSQ_NOALLOC_SCRATCH_BYTES (32u << 20)

int nsq_causal_conv1d_bwd_noalloc(const void* gy, const void* x, const float* weight, const float* bias, void* gx,
                                  float* gweight, float* gbias, int dtype, int activation, int64_t B, int64_t C,
                                  int64_t L, int64_t K, void* stream);

/*
 * Back-to-back striped-Hyena short-conv block ("projection conv, pre-gate,
 * mixer conv with skip, post-gate"; nvsubquadratic/ops/causal_conv1d_custom.py:101-121,
 * which binds subquadratic_ops_torch.b2b_causal_conv1d):
 *   p = causal_conv(x; weight_proj) over 3C channels;  q, k, v = p split in three;
 *   z = k*v;  h = causal_conv(z; weight_mixer) + skip*z;  y = q*h.
 * Both convs use the nn.Conv1d tap order above; fp32 throughout, y rounded once.
 * x, gx: [B, 3C, L]; y, gy: [B, C, L] in `dtype`; weight_proj [3C, Kp],
 * weight_mixer [C, Km], skip_bias [C] float32 (skip may be NULL = 0); gradients
 * float32 of the same shapes (gskip may be NULL).  1 <= Kp, Km <= 256.
 */
int nsq_b2b_causal_conv1d_fwd(const void* x, const float* weight_proj, const float* weight_mixer,
                              const float* skip_bias, void* y, int dtype, int64_t B, int64_t C, int64_t L, int64_t Kp,
                              int64_t Km, void* stream);

size_t nsq_b2b_causal_conv1d_bwd_workspace_bytes(int64_t B, int64_t C, int64_t L, int64_t Kp, int64_t Km);

int nsq_b2b_causal_conv1d_bwd(const void* gy, const void* x, const float* weight_proj, const float* weight_mixer,
                              const float* skip_bias, void* gx, float* gweight_proj, float* gweight_mixer,
                              float* gskip, int dtype, int64_t B, int64_t C, int64_t L, int64_t Kp, int64_t Km,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * Non-causal "same" 2D / 3D FFT convolution (+ shortcut), nd = 2 or 3:
 *   y = crop_{K_d//2}( x (*) k ).to(dtype) + shortcut * x
 * x, y, g, gx: [B, H, S_0, .., S_{nd-1}] in `dtype`; k, gk: [kbatch*H, K_0, ..] float32
 * with kbatch = 1 (shared) or B (per-sample FiLM kernels); shortcut [H] in `dtype`
 * (may be NULL); gs: [kbatch*H] float32 per-kernel-row shortcut-gradient partials
 * (the caller sums over kbatch).  S, K: host arrays of nd sizes, K_d <= 2 S_d, and
 * every axis must fit an FFT length of 1024.
 * Results follow nvsubquadratic/ops/fftconv.py:662-733 (fftconv2d_fp32_bhl) and
 * :736-812 (fftconv3d_fp32_bhl); the 2D call replaces the native kernel bound at
 * nvsubquadratic/ops/fftconv_custom.py:117-125 (subquadratic_ops_torch.fft_conv2d)
 * plus the shortcut epilogue of fftconv2d_bhl (:133-160).  The reference has no
 * native 3D kernel (nvsubquadratic/modules/ckconv_nd.py:721-724).
 */
size_t nsq_fftconv_nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                                      int64_t kbatch, int direction);
/* A forward given a workspace of the backward's size keeps the transformed x
 * and the filter spectrum in it; a backward called on that untouched workspace
 * with fwd_state = 1 reuses them (results identical to fwd_state = 0). */

int nsq_fftconv_nd_fwd(int nd, const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                       int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch, void* workspace,
                       size_t workspace_bytes, void* stream);

int nsq_fftconv_nd_bwd(int nd, const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk,
                       float* gs, int dtype, int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch,
                       void* workspace, size_t workspace_bytes, int fwd_state, void* stream);

/*
 * Circular and mixed-boundary 2D / 3D FFT convolution: the nsq_fftconv_nd_*
 * calls above with a per-axis boundary condition.  Bit d of `periodic` set =
 * axis d is periodic: no padding along it, K_d <= S_d, and
 *   y[.., n_d, ..] = sum_j k[.., j_d, ..] x[.., (n_d + (K_d-1)//2 - j_d) mod S_d, ..]
 * (the circular "same" alignment, shift -((K_d-1)//2) as a phase ramp on the
 * filter spectrum).  Clear bits are zero-padded "same" axes exactly as above.
 * Periodic lengths must be powers of two up to 1024 (NSQ_ERR_UNSUPPORTED
 * otherwise; lengths below 16 run on their periodic extension at 16).  periodic = 0 is nsq_fftconv_nd_*; all bits set is the circular
 * conv.  Replaces nvsubquadratic/ops/circular_fftconv.py:406-483
 * (circular_fftconv2d_fp32_bhl), :486-569 (circular_fftconv3d_fp32_bhl) and
 * nvsubquadratic/ops/mixed_fftconv.py:504-630 (_mixed_fftconv_nd_fp32_bhl,
 * behind mixed_fftconv{2,3}d_fp32_bhl :663-729), which are torch.fft code in
 * the reference (no native kernel to bind).  Workspace and fwd_state as above.
 */
size_t nsq_mixed_fftconv_nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                                            int64_t kbatch, unsigned periodic, int direction);

int nsq_mixed_fftconv_nd_fwd(int nd, const void* x, const float* k, const void* shortcut, void* y, int dtype,
                             int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch,
                             unsigned periodic, void* workspace, size_t workspace_bytes, void* stream);

int nsq_mixed_fftconv_nd_bwd(int nd, const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                             float* gk, float* gs, int dtype, int64_t B, int64_t H, const int64_t* S,
                             const int64_t* K, int64_t kbatch, unsigned periodic, void* workspace,
                             size_t workspace_bytes, int fwd_state, void* stream);

/* ---------------------------------------------------------------------------
 * Implicit filter generation (SIREN MLP): the hidden stack (ABI 9).
 *
 * Replaces the hidden layers of nvsubquadratic/modules/kernels_nd.py:1149-1190
 * (SIRENKernelND.forward without FiLM: the positional embedding and the
 * sine-activated stack):
 *   a_0[g] = sin(W0 x_g + b0)                       W0 [E, d], b0 [E]
 *   a_i[g] = sin(W_i a_{i-1}[g] + b_i), i = 1..nh   W_1 [HD, E], W_i [HD, HD]
 * for the G coordinates grid [G, d] (d = 1..3).  The forward writes
 * act [HD + 1][lda] fp32 = [a_nh^T; 1]: the last activation transposed with a
 * row of ones, so that the reference's readout k = W_out a_nh + b_out becomes
 * one library GEMM [W_out | b_out] act writing the filter straight in the
 * [H][G] layout the FFT convs read (the rearrange of modules/ckconv_nd.py:
 * 1149-1164 never materialises).  The hidden weights are packed back to back in
 * wh (W_1, W_2, ...), their biases in bh.  Bias pointers may be null
 * (use_bias=False).  E, HD in {16, 32, 64, 128}; 1 <= nh <= 8.  fp32
 * throughout, matrix cores for the products (fp32 in, fp32 accumulate).  Other
 * sizes: NSQ_ERR_UNSUPPORTED.
 *
 * Backward: gact = dL/da_nh (= W_out^T gk, from the readout's gradient GEMM)
 * in, element (j, g) at gact[j * gact_stride_j + g * gact_stride_g] (so both
 * [HD][G] and [G][HD] layouts read in place); the gradients of W0, b0, wh, bh
 * out (gb0 / gbh may be null when the biases are).  The layers are recomputed from the grid (no
 * forward state); partial sums go to the workspace and are reduced in a fixed
 * order (deterministic).
 */
int nsq_siren_mlp_fwd(const float* grid, int64_t G, int d, const float* w0, const float* b0, int E, const float* wh,
                      const float* bh, int nh, int HD, float* act, int64_t lda, void* stream);

/* Readout of the same generator (kernels_nd.py:1189, SIRENKernelND's output
 * linear): k[h][g] = b_out[h] + W_out[h] . a_nh[g] for W_out [H, HD], b_out [H]
 * (may be null), act rows 0..HD-1 of nsq_siren_mlp_fwd's output (row stride
 * lda), written as k [H][G] fp32: the filter in the layout the FFT convs read.
 * HD in {16, 32, 64, 128}. */
int nsq_siren_readout_fwd(const float* wout, const float* bout, int64_t H, int HD, const float* act, int64_t lda,
                          int64_t G, float* k, void* stream);

/* The readout's gradients in one pass over gk (ABI 11; the reference gets them
 * from autograd of SIRENKernelND's out_linear, kernels_nd.py:1189, two GEMMs
 * that each read the filter gradient):
 *   gact[s][j][g] = sum_h W_out[h][j] gk[s][h][g]          ([nb][HD][G], row stride G)
 *   gwout[h][j]   = sum_s sum_g gk[s][h][g] act[s][j][g]   ([H][HD])
 *   gbout[h]      = sum_s sum_g gk[s][h][g]                ([H]; may be null)
 * for nb samples s (1 for a shared filter): gk [nb][H][ldk], act [nb][HD + 1][lda]
 * (nsq_siren_mlp_fwd's output; row HD is not read).  The products run on the bf16
 * matrix cores with both operands split into bf16 halves (three products per step,
 * fp32 accumulation: ~2^-17 relative error per product); partial sums are reduced
 * in a fixed order (deterministic).  HD in {16, 32, 64}; 128 returns
 * NSQ_ERR_UNSUPPORTED (the caller keeps library GEMMs there).  gact feeds
 * nsq_siren_mlp_bwd with gact_stride_j = G, gact_stride_g = 1. */
size_t nsq_siren_readout_bwd_workspace_bytes(int64_t H, int HD, int64_t G, int64_t nb);

int nsq_siren_readout_bwd(const float* gk, int64_t ldk, const float* act, int64_t lda, const float* wout, int64_t H,
                          int HD, int64_t G, int64_t nb, float* gact, float* gwout, float* gbout, void* workspace,
                          size_t workspace_bytes, void* stream);

size_t nsq_siren_mlp_bwd_workspace_bytes(int64_t G, int d, int E, int nh, int HD);

int nsq_siren_mlp_bwd(const float* gact, int64_t gact_stride_j, int64_t gact_stride_g, const float* grid, int64_t G,
                      int d, const float* w0, const float* b0, int E, const float* wh, const float* bh, int nh, int HD,
                      float* gw0, float* gb0, float* gwh, float* gbh, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Causal 1D FFT convolution with a SIREN filter that is never formed (ABI 14):
 * CKConvND's causal path (nvsubquadratic/modules/ckconv_nd.py:1149-1164 with an
 * identity mask: the SIRENKernelND filter k = W_out a + b_out of kernels_nd.py:
 * 1181-1189 at its causal points, then the causal conv of ops/fftconv.py:546-600,
 * the job nsq_siren_readout_fwd + nsq_fftconv1d_causal_fwd do with k in HBM):
 *   y[b,h,:] = causal_conv(x[b,h,:]; k_h) + shortcut[h] x[b,h,:],
 *   k_h[g] = sum_{j<HD} wout[h][j] act[j][g] + bout[h],  g < K,
 * for act [HD + 1][lda] (nsq_siren_mlp_fwd's output: row HD is the ones row and
 * must hold ones), wout [H][HD], bout [H] or NULL, x / y / g / gx [B, H, L] in
 * `dtype`, shortcut [H] or NULL.  The 4-step plan's column pass is linear, so
 * the forward transforms the HD + 1 activation rows once and forms each
 * channel's filter transform from them (fp32, fixed order); the backward reads
 * the filter gradient's spectrum once for gwout, gbout and wout^T times it (the
 * inverse column pass's adjoint is the forward one / N) and inverse-transforms
 * only those HD rows into gact [HD][K] (row stride K; feeds nsq_siren_mlp_bwd
 * with gact_stride_j = K, gact_stride_g = 1).  gs [H] (fp32, required with a
 * shortcut) is the shortcut gradient; gbout may be NULL.  The gradient products
 * run as in nsq_siren_readout_bwd (bf16-split matrix cores, fp32 accumulation,
 * fixed-order sums).  Results equal the composition's to fp32 rounding.
 * Takes the 4-step plan only: FFT lengths 2^15 .. 2^23 (L + K above 16384,
 * K <= L + 1) with HD in {16, 32, 64}; other shapes return NSQ_ERR_UNSUPPORTED
 * (the fused plan reads the filter: form it with nsq_siren_readout_fwd).
 * Workspace (one size, both directions; 256-byte aligned): the forward leaves
 * the transformed x, filter and activations there, and the backward with
 * fwd_state = 1 starts from them (untouched since that forward); fwd_state = 0
 * recomputes them.  No counterpart in the reference: there the filter is a
 * torch tensor between the generator and the conv. */
size_t nsq_siren_fftconv1d_causal_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int HD);

int nsq_siren_fftconv1d_causal_fwd(const void* x, const float* act, int64_t lda, const float* wout,
                                   const float* bout, int HD, const void* shortcut, void* y, int dtype, int64_t B,
                                   int64_t H, int64_t L, int64_t K, void* workspace, size_t workspace_bytes,
                                   void* stream);

int nsq_siren_fftconv1d_causal_bwd(const void* g, const void* x, const float* act, int64_t lda, const float* wout,
                                   const float* bout, int HD, const void* shortcut, void* gx, float* gact,
                                   float* gwout, float* gbout, float* gs, int dtype, int64_t B, int64_t H, int64_t L,
                                   int64_t K, void* workspace, size_t workspace_bytes, int fwd_state, void* stream);

/* FiLM-conditioned generator (ABI 12): kernels_nd.py:1165-1187 with the
 * KernelFiLMGenerator output of modules/film.py:75 (its MLP runs on the
 * caller's side; these take its (gamma, beta) pairs).  film [nb][nfilm][2][HD]
 * fp32: for sample s and FiLM slot f, gamma = film[s][f][0], beta =
 * film[s][f][1]; slot f modulates h = gamma * sin(z) + beta at the output of
 * hidden layer f + 1 - film_first, and with film_first (film_after_pos_embed,
 * needs E == HD) slot 0 modulates the positional embedding; nfilm = nh +
 * film_first.  The filter becomes per sample:
 *   nsq_siren_mlp_film_fwd      act [nb][HD + 1][lda] (sample s's rows at s (HD + 1) lda);
 *   nsq_siren_film_readout_fwd  k [nb][H][G] from that act (also the plain readout's batched form);
 *   nsq_siren_mlp_film_bwd      gact element (s, j, g) at s gact_stride_s + j gact_stride_j + g gact_stride_g
 *                               (nsq_siren_readout_bwd's [nb][HD][G] output reads in place); the weight and bias
 *                               gradients summed over the samples, gfilm [nb][nfilm][2][HD] per sample.
 * film = null with nb = 1 and film_first = 0 is the plain generator (the entry
 * points above are exactly that).  Deterministic, fixed-order reductions. */
int nsq_siren_mlp_film_fwd(const float* grid, int64_t G, int d, const float* w0, const float* b0, int E,
                           const float* wh, const float* bh, int nh, int HD, const float* film, int64_t nb,
                           int film_first, float* act, int64_t lda, void* stream);

int nsq_siren_film_readout_fwd(const float* wout, const float* bout, int64_t H, int HD, const float* act,
                               int64_t lda, int64_t G, int64_t nb, float* k, void* stream);

size_t nsq_siren_mlp_film_bwd_workspace_bytes(int64_t G, int d, int E, int nh, int HD, int64_t nb, int film_first);

int nsq_siren_mlp_film_bwd(const float* gact, int64_t gact_stride_j, int64_t gact_stride_g, int64_t gact_stride_s,
                           const float* grid, int64_t G, int d, const float* w0, const float* b0, int E,
                           const float* wh, const float* bh, int nh, int HD, const float* film, int64_t nb,
                           int film_first, float* gw0, float* gb0, float* gwh, float* gbh, float* gfilm,
                           void* workspace, size_t workspace_bytes, void* stream);

/* QK-norm over channels (ABI 13): nvsubquadratic/utils/qk_norm.py L2Norm, i.e.
 * F.normalize(x, p=2, dim=channels, eps) at the Hyena operator's q / k norm site
 * (modules/hyena_nd.py:529-543): out[b,c,s] = round(x / max(round(||x[b,:,s]||), eps)),
 * the norm over the C channels accumulated in fp32 and rounded to the I/O dtype
 * as torch's norm of a 16-bit tensor is.  x [B, C, S] channels-first; out
 * [B, S, C] (out_channels_last) or [B, C, S]; the backward's dout has the output's
 * layout and dx the input's: dx = (dout - xhat sum_c(dout xhat)) / n, dout / n
 * where n was clamped.  One pass each way, no workspace.  C <= 7781 forward,
 * C <= 3536 backward (NSQ_ERR_UNSUPPORTED beyond). */
int nsq_channel_l2norm_fwd(const void* x, void* out, int dtype, int64_t B, int64_t C, int64_t S, float eps,
                           int out_channels_last, void* stream);

int nsq_channel_l2norm_bwd(const void* dout, const void* x, void* dx, int dtype, int64_t B, int64_t C, int64_t S,
                           float eps, int out_channels_last, void* stream);

/* ---------------------------------------------------------------------------
 * Channels-last (BLH) layout changes (ABI 9).
 *
 * dst[b][c][r] = src[b][r][c] for B matrices of R x C elements of elem_bytes
 * (2: bf16 / fp16, 4: fp32) bytes.  Replaces the materialised
 * rearrange("b l h -> b h l") of the `_w_reshape` / `_blh` wrappers
 * (nvsubquadratic/ops/fftconv.py:163-232, 449-538; ops/fftconv_custom.py:338-359),
 * and its inverse with R and C swapped.  src and dst must not alias.
 */
int nsq_batched_transpose(const void* src, void* dst, int elem_bytes, int64_t B, int64_t R, int64_t C,
                          void* stream);

/* ---------------------------------------------------------------------------
 * Hyena gate + RMSNorm over channels + layout, one pass (ABI 10).
 *
 * Replaces, per call, the reference's chain of elementwise ops and copies
 *   u = y * act(v)                              (hyena_nd.py:570; :546 for gate 1)
 *   out = RMSNorm(u.movedim(1, -1))             (hyena_nd.py:573-580 output_norm;
 *         rms_norm.py:71-77: fp32 upcast, u * rsqrt(mean_c u^2 + eps),
 *         (w * .).to(dtype); rms_norm_channel_first.py:71-80 along dim 1)
 *   rearrange(out, "b c ... -> b ... c")        (hyena_nd.py:583)
 * y, v: [B, C, S] in `dtype` (S = the flattened spatial axes); v == NULL skips
 * the gate (u = y).  w: fp32 [C].  out_channels_last = 1 writes out as
 * [B, S, C] (the output_norm site), 0 as [B, C, S] (the pixelhyena_norm site,
 * hyena_nd.py:548-556).  act: NSQ_GATE_*.  C <= 7781 (forward), C <= 3536
 * (backward); larger C returns NSQ_ERR_UNSUPPORTED.
 *
 * Backward: dout in the forward's output layout; writes dy (and dv when v is
 * given; v and dv come together) as [B, C, S] and dw fp32 [C] (overwritten,
 * summed in a fixed order).  Workspace: nsq_channel_rmsnorm_bwd_workspace_bytes
 * (per-workgroup partial rows of dw).
 */
int nsq_channel_rmsnorm_fwd(const void* y, const void* v, const float* w, void* out, int dtype, int64_t B, int64_t C,
                            int64_t S, float eps, int act, int out_channels_last, void* stream);

size_t nsq_channel_rmsnorm_bwd_workspace_bytes(int64_t B, int64_t C, int64_t S);

int nsq_channel_rmsnorm_bwd(const void* dout, const void* y, const void* v, const float* w, void* dy, void* dv,
                            float* dw, int dtype, int64_t B, int64_t C, int64_t S, float eps, int act,
                            int out_channels_last, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Hyena gate + LayerNorm over channels + layout, one pass (ABI 15).
 *
 * The pixelhyena_norm site with a torch.nn.LayerNorm(C) module (the reference's
 * configs' other norm there, e.g. examples/imagenet_classification/
 * ccnn_7_512_hyena.py: LazyConfig(torch.nn.LayerNorm)(normalized_shape=...)),
 * which hyena_nd.py:548-556 applies to z = q * act(k) moved to channels-last
 * and flattened: per position over the C channels,
 *   mu = mean_c u, var = mean_c (u - mu)^2 (biased),
 *   out = round(w[c] ((u - mu) rsqrt(var + eps)) + b[c])   (fp32 arithmetic)
 * with u = round(y * round(act(v))) (v == NULL: u = y).  Same layouts and
 * arguments as nsq_channel_rmsnorm_*; w and b (fp32 [C]) may be NULL (no
 * elementwise affine: scale 1, shift 0).  C <= 7781 forward, C <= 3241
 * backward (NSQ_ERR_UNSUPPORTED beyond).
 *
 * Backward: writes dy (and dv with v), and dw / db (fp32 [C], overwritten,
 * summed in a fixed order) when given; dw needs w.  Workspace:
 * nsq_channel_layernorm_bwd_workspace_bytes (partial rows of dw and db; none
 * needed when dw and db are both NULL).
 */
int nsq_channel_layernorm_fwd(const void* y, const void* v, const float* w, const float* b, void* out, int dtype,
                              int64_t B, int64_t C, int64_t S, float eps, int act, int out_channels_last,
                              void* stream);

size_t nsq_channel_layernorm_bwd_workspace_bytes(int64_t B, int64_t C, int64_t S);

int nsq_channel_layernorm_bwd(const void* dout, const void* y, const void* v, const float* w, void* dy, void* dv,
                              float* dw, float* db, int dtype, int64_t B, int64_t C, int64_t S, float eps, int act,
                              int out_channels_last, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Hyena gate + GroupNorm over channels, channels-first (ABI 16).
 *
 * The pixelhyena_norm site with a torch.nn.GroupNorm(num_groups, C) module
 * (the reference's configs use num_groups = 1, e.g.
 * examples/imagenet_classification/ccnn_7_512_hyena.py), which hyena_nd.py:
 * 548-550 applies channels-first (modules/_channels_first_utils.py:27) to
 * z = q * act(k): per sample b and group g of C / G consecutive channels, over
 * those channels and all S positions,
 *   mu, var = mean and biased variance of u,  r = rsqrt(var + eps),
 *   out[b,c,s] = round(u a + h),  a = r w[c],  h = b[c] - mu a
 * (fp32 arithmetic; torch's scale / shift form) with u = round(y *
 * round(act(v))) (v == NULL: u = y).  y, v, out: [B, C, S] of dtype; w, b:
 * fp32 [C] or NULL (scale 1, shift 0).  mean and rstd (fp32 [B, G]) receive
 * mu and r, which the backward takes.  C must be a multiple of G.  Workspace:
 * nsq_channel_groupnorm_workspace_bytes(B, C, G, NSQ_DIR_FWD).
 *
 * Backward: writes dy (and dv with v) as [B, C, S] and dw / db (fp32 [C],
 * overwritten, summed in a fixed order) when given; dw needs w.  Workspace:
 * nsq_channel_groupnorm_workspace_bytes(B, C, G, NSQ_DIR_BWD).
 */
size_t nsq_channel_groupnorm_workspace_bytes(int64_t B, int64_t C, int64_t G, int direction);

int nsq_channel_groupnorm_fwd(const void* y, const void* v, const float* w, const float* b, void* out, float* mean,
                              float* rstd, int dtype, int64_t B, int64_t C, int64_t S, int64_t G, float eps, int act,
                              void* workspace, size_t workspace_bytes, void* stream);

int nsq_channel_groupnorm_bwd(const void* dout, const void* y, const void* v, const float* w, const float* mean,
                              const float* rstd, void* dy, void* dv, float* dw, float* db, int dtype, int64_t B,
                              int64_t C, int64_t S, int64_t G, int act, void* workspace, size_t workspace_bytes,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSQ_HIP_H_ */

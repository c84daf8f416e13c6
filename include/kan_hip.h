/*
 * kan_hip.h -- C-ABI of libkan_hip.so, the gfx950 (MI355X) kernels behind the
 * KANLinear hot path of torch-spline-kan.
 *
 * Every entry point takes raw device pointers, int64 sizes, a dtype code and
 * a hipStream_t (passed as void*; NULL = legacy default stream), launches its
 * kernels asynchronously on that stream and returns a status code.  No entry
 * point allocates device memory: outputs and workspaces are provided by the
 * caller (the workspace-size queries say how large).  On a non-zero status,
 * kan_hip_last_error() returns a message for the calling thread.  Invalid
 * sizes are rejected before any launch, so an error never leaves a kernel
 * behind.
 *
 * Layouts are row-major and contiguous:
 *   x [n, I]; grid [I, G+2k+1]; base_weight [O, I]; spline_weight [O, I, R];
 *   spline_scaler [O, I]; basis [n, I, R]; output [n, O]; with R = G + k.
 * The "augmented basis" is [n, W] with W = kan_hip_aug_width(I, G, k, base):
 *   row n = [ basis(n, 0, 0..R-1), ..., basis(n, I-1, ..), silu(x(n, 0..I-1)), pad ]
 * (the silu block only when a base branch is present).  It is produced by the
 * forward and consumed by the backward.
 *
 * Reference interfaces each entry point replaces are cited per function
 * (paths relative to the torch-spline-kan source tree).
 */
#ifndef KAN_HIP_H_
#define KAN_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define KAN_DTYPE_F32 0
#define KAN_DTYPE_F64 1

/* status codes */
#define KAN_OK 0
#define KAN_ERR_INVALID 1  /* bad argument (shape, dtype code, null pointer) */
#define KAN_ERR_LIMIT 2    /* configuration outside the native kernel limits */
#define KAN_ERR_HIP 3      /* HIP runtime error at launch */
#define KAN_ERR_WORKSPACE 4 /* workspace too small */

/* Message for the last non-zero status returned on this thread ("" if none). */
const char* kan_hip_last_error(void);

/* Hex digest of the sources and compiler flags the library was built from
 * (no reference counterpart: the loader uses it to refuse a library that is
 * older than the sources beside it). */
const char* kan_hip_source_hash(void);

/* Limits query.  Replaces the module attributes CUDA_MAX_DEG0_BASIS and
 * CUDA_MAX_IN_FEATURES (csrc/kan_ext.cpp:164-165, csrc/kan_ops.h:15-17). */
int kan_hip_limits(int64_t* max_deg0_basis, int64_t* max_in_features);

/* Basis implementation switch: 0 = dense Cox-de Boor recurrence, 1 = local
 * (default).  Replaces _C.set_basis_impl / _C.get_basis_impl
 * (csrc/kan_cuda.cu:274-279, csrc/kan_ext.cpp:193-195).  Any other value
 * returns KAN_ERR_INVALID. */
int kan_hip_set_basis_impl(int64_t impl);
int64_t kan_hip_get_basis_impl(void);

/* Routing switches of the native path (no reference counterpart: they choose
 * between kernel routes that give the same results, for tests and tuning).
 * Each starts from its environment variable, read once when the library is
 * loaded; kan_hip_set_route changes it for the whole process.  A workspace
 * query and the launch it sizes must see the same routes.
 *   KAN_ROUTE_FUSED_DX   (KAN_HIP_FUSED_DX)   0 off (default), 1 dx contracted
 *                        in the input-side product's epilogue
 *   KAN_ROUTE_COMPACT_E  (KAN_HIP_COMPACT_E)  -1 automatic (R >= 25, default),
 *                        0 never, 1 always: span-window form of E
 *   KAN_ROUTE_EDGE_FUSED (KAN_HIP_EDGE_FUSED) 1 (default) both gradient sides
 *                        of the edge statistic in one kernel, 0 separate
 *   KAN_ROUTE_GEMM_TILE  (KAN_HIP_GEMM_TILE)  -1 cost model (default), 0 256x256
 *                        ("256"), 1 128x128 ("128"), 2 256x64 ("256x64"),
 *                        3 4-wave 256x256 ("256w4"); float64 products take
 *                        0 as 256x128, 1 as 128x128, 2 as the pipelined
 *                        128x128 tile with 32-deep slabs and 3 as the
 *                        pipelined 64x64 tile
 * kan_hip_set_route returns KAN_ERR_INVALID for an unknown route or value;
 * kan_hip_get_route returns -2 for an unknown route. */
#define KAN_ROUTE_FUSED_DX 0
#define KAN_ROUTE_COMPACT_E 1
#define KAN_ROUTE_EDGE_FUSED 2
#define KAN_ROUTE_GEMM_TILE 3
#define KAN_ROUTE_COUNT 4
int kan_hip_set_route(int route, int value);
int kan_hip_get_route(int route);

/* basis[n, I, R] = B-spline basis of x.  Replaces _C.basis / kan_basis_cuda
 * (csrc/kan_ext.cpp:196-197, csrc/kan_cuda.cu:666-680). */
int kan_hip_basis(int dtype, const void* x, const void* grid, void* basis, int64_t n,
                  int64_t in_features, int64_t grid_size, int64_t spline_order, void* stream);

/* grad_x[n, i] = sum_r grad_basis[n, i, r] * dB_r/dx(x[n, i]).  Replaces
 * _C.basis_grad / kan_basis_grad_cuda (csrc/kan_ext.cpp:198-200,
 * csrc/kan_cuda.cu:682-699). */
int kan_hip_basis_grad(int dtype, const void* x, const void* grid, const void* grad_basis,
                       void* grad_x, int64_t n, int64_t in_features, int64_t grid_size,
                       int64_t spline_order, void* stream);

/* basis[n, I, R] and silu[n, I] = x * sigmoid(x) in one pass over x: the two
 * operands that forward_with_regularization's native path takes from
 * base_activation (SiLU) and the native basis separately
 * (spline_kan/kan_linear.py:380-381; the native path requires SiLU,
 * kan_linear.py:213). */
int kan_hip_basis_silu(int dtype, const void* x, const void* grid, void* basis, void* silu,
                       int64_t n, int64_t in_features, int64_t grid_size, int64_t spline_order,
                       void* stream);

/* grad_x[n, i] = sum_r grad_basis[n, i, r] * dB_r/dx(x[n, i])
 *              + grad_silu[n, i] * silu'(x[n, i]): the gradients that autograd
 * takes through the basis and SiLU of those call sites and adds, in one
 * pass. */
int kan_hip_basis_silu_grad(int dtype, const void* x, const void* grid, const void* grad_basis,
                            const void* grad_silu, void* grad_x, int64_t n, int64_t in_features,
                            int64_t grid_size, int64_t spline_order, void* stream);

/* out[n, i, r] = scale[n, i] * d^order B_r / dx^order at x[n, i] (order >= 0;
 * order 0 is the basis itself, order > spline_order gives zeros; scale may be
 * NULL for 1), with the span, boundary and zero-denominator conventions of
 * kan_hip_basis.  Replaces the differentiable basis derivatives that the
 * reference builds from ATen ops when the backward is recorded
 * (create_graph=True): compute_basis_derivative
 * (spline_kan/reference_backend.py:99-125) and autograd through
 * compute_basis (reference_backend.py:69-94), as used by
 * kan_backward_composite (csrc/kan_cpu.cpp:301-345) and NativeBasis
 * (spline_kan/fused.py:57-60); the scale folds the elementwise product the
 * recorded backward applies to them (g * D^q B). */
int kan_hip_basis_deriv(int dtype, const void* x, const void* grid, const void* scale, void* out,
                        int64_t n, int64_t in_features, int64_t grid_size, int64_t spline_order,
                        int64_t order, void* stream);

/* grad_x[n, i] = scale[n, i] * (sum_r grad_basis[n, i, r] * d^order B_r/dx^order(x[n, i])
 *                + grad_base[n, i] * silu^(order)(x[n, i]))
 * (order 1 without base or scale is kan_hip_basis_grad; grad_base and scale
 * may be NULL; with grad_base, order <= 4).  The contraction behind the
 * higher-order derivatives of the same reference call sites, without forming
 * the derivative tensor; the base term is the SiLU branch of
 * kan_backward_composite (csrc/kan_cpu.cpp:335-342) and its derivatives. */
int kan_hip_basis_deriv_contract(int dtype, const void* x, const void* grid,
                                 const void* grad_basis, const void* grad_base,
                                 const void* scale, void* grad_x, int64_t n,
                                 int64_t in_features, int64_t grid_size, int64_t spline_order,
                                 int64_t order, void* stream);

/* out[e] = scale[e] * silu^(order)(x[e]) for count elements (order 0..4;
 * scale may be NULL).  The SiLU terms of the recorded backward (silu(x) and
 * silu'(x) of kan_backward_composite, csrc/kan_cpu.cpp:335-342, and their
 * derivatives) as one launch each. */
int kan_hip_silu_deriv(int dtype, const void* x, const void* scale, void* out, int64_t count,
                       int64_t order, void* stream);

/* C[M, N] = op(A) op(B) on the MFMA contraction engine, for the products
 * of the recorded (create_graph=True) backward.  op(A) is A [M, K] with row
 * stride lda (trans_a = 0) or the transpose of A stored [K, M] (trans_a = 1);
 * op(B) is B [K, N] (trans_b = 0) or the transpose of B stored [N, K]
 * (trans_b = 1); C is [M, N] with row stride ldc.  Products with a long K
 * and few output tiles (sample reductions such as D^T H) are split over K
 * into partial slices in ws and summed in a fixed order, so results are
 * deterministic.  Replaces the torch::mm calls of kan_backward_composite
 * (csrc/kan_cpu.cpp:322-343) and the matmuls autograd records through them.
 * kan_hip_matmul_workspace gives the ws size in bytes (0 when no split). */
int kan_hip_matmul_workspace(int dtype, int trans_a, int trans_b, int64_t M, int64_t N,
                             int64_t K, size_t* bytes);
int kan_hip_matmul(int dtype, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                   const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                   void* ws, size_t ws_bytes, void* stream);

/* Inference path (no saved basis).  kan_hip_pack_weight writes the packed
 * weight waug [O, ld] = [spline_weight * spline_scaler | base_weight] once;
 * an inference caller keeps it while the parameters do not change (the
 * folding that export_inference performs, spline_kan/kan_linear.py:471-496).
 * kan_hip_infer then computes output [n, O] from x with that weight: the
 * augmented basis lives only in the caller's workspace, and products with
 * few output tiles (small batches) are split over K and summed in a fixed
 * order.  Same output as kan_hip_forward (csrc/kan_cuda.cu:469-532) up to
 * the summation order of split products.  kan_hip_infer_workspace sizes ws. */
int kan_hip_pack_weight(int dtype, const void* base_weight, const void* spline_weight,
                        const void* spline_scaler, void* weight_aug, int64_t in_features,
                        int64_t out_features, int64_t grid_size, int64_t spline_order,
                        void* stream);
int kan_hip_infer_workspace(int dtype, int64_t n, int64_t in_features, int64_t out_features,
                            int64_t grid_size, int64_t spline_order, int has_base, size_t* bytes);
int kan_hip_infer(int dtype, const void* x, const void* grid, const void* weight_aug, void* output,
                  void* ws, size_t ws_bytes, int64_t n, int64_t in_features, int64_t out_features,
                  int64_t grid_size, int64_t spline_order, int has_base, void* stream);

/* Allocation-free inference.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, kernels
 * and result as kan_hip_infer, without the workspace: the library uses a
 * fixed device scratch of KAN_NOALLOC_SCRATCH_BYTES per GPU (held from the
 * library's load until the process ends) and calls no allocating routine.
 * A call whose workspace (kan_hip_infer_workspace) exceeds that size
 * returns KAN_ERR_WORKSPACE before any launch.  All calls on one GPU share
 * its scratch: calls that overlap in time on one GPU (other streams, other
 * threads) race and must be serialised by the caller.  The calling
 * thread's current device must be the one the pointers and the stream
 * belong to. */
#define KAN_NOALLOC_SCRATCH_BYTES (64u * 1024u * 1024u)
int kan_hip_infer_noalloc(int dtype, const void* x, const void* grid, const void* weight_aug,
                          void* output, int64_t n, int64_t in_features, int64_t out_features,
                          int64_t grid_size, int64_t spline_order, int has_base, void* stream);

/* Row width (elements) of the augmented basis and augmented weight buffers.
 * Returns -1 for invalid sizes.  No reference counterpart: the reference keeps
 * basis [n, I, R] and runs the SiLU branch as a second GEMM
 * (csrc/kan_cuda.cu:521-531). */
int64_t kan_hip_aug_width(int64_t in_features, int64_t grid_size, int64_t spline_order,
                          int has_base);

/* Forward: output = silu(x) base_weight^T + basis(x) (spline_weight*scaler)^T.
 * base_weight may be NULL (no fused base branch), spline_scaler may be NULL
 * (no scaler).  Writes output [n, O] and basis_aug [n, W] (kept for
 * backward).  The workspace holds the augmented weight [O, W] and, for
 * products with few output tiles (few samples or outputs against a long
 * K), the split-K partial slices of the output, summed in a fixed order;
 * kan_hip_forward_workspace gives its size.  Replaces kan_forward_cuda
 * (csrc/kan_cuda.cu:469-532) behind _C.kan_forward / KANFunction::forward
 * (csrc/kan_ext.cpp:10-33, csrc/kan_autograd.cpp:18-47). */
int kan_hip_forward_workspace(int dtype, int64_t n, int64_t in_features, int64_t out_features,
                              int64_t grid_size, int64_t spline_order, int has_base,
                              size_t* bytes);
int kan_hip_forward(int dtype, const void* x, const void* grid, const void* base_weight,
                    const void* spline_weight, const void* spline_scaler, void* output,
                    void* basis_aug, void* workspace, size_t workspace_bytes, int64_t n,
                    int64_t in_features, int64_t out_features, int64_t grid_size,
                    int64_t spline_order, void* stream);

/* Builds basis_aug [n, W] from a caller-held basis [n, I, R] and x (silu block
 * only when has_base).  Used by the raw backward op, whose caller passes the
 * basis returned by the forward (csrc/kan_ext.cpp:35-56). */
int kan_hip_pack_basis(int dtype, const void* basis, const void* x, void* basis_aug, int64_t n,
                       int64_t in_features, int64_t grid_size, int64_t spline_order,
                       int has_base, void* stream);

/* Workspace bytes kan_hip_backward needs for the given requests. */
int kan_hip_backward_workspace(int dtype, int64_t n, int64_t in_features, int64_t out_features,
                               int64_t grid_size, int64_t spline_order, int has_base,
                               int need_x, int need_params, size_t* bytes);

/* First-order backward.  Each output pointer may be NULL when not requested:
 *   grad_x [n, I], grad_base_weight [O, I], grad_spline_weight [O, I, R],
 *   grad_spline_scaler [O, I] (requires grad_spline_weight's GEMM, computed
 *   together).  Replaces kan_backward_cuda_ex (csrc/kan_cuda.cu:537-630)
 * behind _C.kan_backward and KANFunction::backward
 * (csrc/kan_ext.cpp:35-56, csrc/kan_autograd.cpp:48-111). */
int kan_hip_backward(int dtype, const void* grad_output, const void* x, const void* grid,
                     const void* base_weight, const void* spline_weight,
                     const void* spline_scaler, const void* basis_aug, void* grad_x,
                     void* grad_base_weight, void* grad_spline_weight, void* grad_spline_scaler,
                     void* workspace, size_t workspace_bytes, int64_t n, int64_t in_features,
                     int64_t out_features, int64_t grid_size, int64_t spline_order,
                     void* stream);

/* Workspace bytes for the edge statistic (backward != 0: backward pass).  The
 * two passes split the samples differently, so each call needs the size
 * queried for its own pass. */
int kan_hip_edge_workspace(int dtype, int64_t n, int64_t in_features, int64_t out_features,
                           int64_t num_basis, int backward, size_t* bytes);

/* a[o, i] = (1/n) sum_m | s[m,i] bw[o,i] + sum_r basis[m,i,r] weight[o,i,r] |
 * without materialising the [n, O, I] edge tensor.  s and base_weight may both
 * be NULL (no base branch).  Replaces _C.edge_abs_mean / edge_abs_mean_cuda
 * (csrc/kan_ext.cpp:201-203, csrc/kan_reg_cuda.cu:263-280). */
int kan_hip_edge_abs_mean(int dtype, const void* s, const void* basis, const void* base_weight,
                          const void* weight, void* a, void* workspace, size_t workspace_bytes,
                          int64_t n, int64_t in_features, int64_t out_features,
                          int64_t num_basis, void* stream);

/* Backward of kan_hip_edge_abs_mean given grad_a [O, I]; each output may be
 * NULL when not needed: grad_s [n, I], grad_basis [n, I, R],
 * grad_base_weight [O, I], grad_weight [O, I, R].  Replaces
 * _C.edge_abs_mean_backward / edge_abs_mean_backward_cuda
 * (csrc/kan_ext.cpp:204-207, csrc/kan_reg_cuda.cu:284-312). */
int kan_hip_edge_abs_mean_backward(int dtype, const void* grad_a, const void* s,
                                   const void* basis, const void* base_weight,
                                   const void* weight, void* grad_s, void* grad_basis,
                                   void* grad_base_weight, void* grad_weight, void* workspace,
                                   size_t workspace_bytes, int64_t n, int64_t in_features,
                                   int64_t out_features, int64_t num_basis, void* stream);

/* Backward of one regularised layer's output and edge statistic together.
 * The layer output y = s bw^T + H W^T (flattened over I and R) and the edge
 * statistic a[o,i] = (1/n) sum_m |phi[m,o,i]| share their operands; with
 * grad_y = dL/dy [n, O] and grad_a = dL/da [O, I] every gradient is one
 * contraction of g'[m,o,i] = grad_a[o,i] sign(phi[m,o,i]) / n + grad_y[m,o]:
 *   grad_s  = sum_o g' bw,   grad_H  = sum_o g' W      (any may be NULL)
 *   grad_bw = sum_m g' s,    grad_W  = sum_m g' H.
 * The reference takes these as the separate F.linear gradients plus
 * EdgeAbsMean's backward, which autograd adds (spline_kan/kan_linear.py:
 * 384-387, spline_kan/fused.py:73-102, csrc/kan_reg_cuda.cu:284-312); here
 * they come from the fused edge kernel with grad_y added to g, with no
 * separate products (with grad_s and grad_basis both NULL, from the
 * parameter kernel with grad_y added alike).  float32 only, for
 * 0 < out_features <= 512,
 * num_basis + 1 <= 16 and n > 0 (kan_hip_edge_linear_supported returns 1
 * exactly then).  Workspace: as kan_hip_edge_abs_mean_backward
 * (kan_hip_edge_workspace with backward = 1). */
int kan_hip_edge_linear_supported(int dtype, int64_t n, int64_t in_features,
                                  int64_t out_features, int64_t num_basis);
int kan_hip_edge_linear_backward(int dtype, const void* grad_a, const void* grad_y, const void* s,
                                 const void* basis, const void* base_weight, const void* weight,
                                 void* grad_s, void* grad_basis, void* grad_base_weight,
                                 void* grad_weight, void* workspace, size_t workspace_bytes,
                                 int64_t n, int64_t in_features, int64_t out_features,
                                 int64_t num_basis, void* stream);

/* Forward of one regularised layer's output and edge statistic together:
 * y [n, O] = s bw^T + H W^T (flattened over I and R) and a [O, I] =
 * (1/n) sum_m |phi[m,o,i]|.  The output is the sum over features of the
 * edge values, y[m,o] = sum_i phi[m,o,i], so one pass over phi gives both.
 * Replaces the two F.linear calls and EdgeAbsMean's forward of
 * forward_with_regularization (spline_kan/kan_linear.py:384-387,
 * spline_kan/fused.py:64-73, csrc/kan_reg_cuda.cu:34-109), which form phi's
 * products twice.  float32, n, in_features, out_features > 0,
 * num_basis + 1 <= 16 (kan_hip_edge_linear_forward_supported returns 1
 * exactly then); s and base_weight both given or both NULL.  Workspace
 * (partial sums of a per 128 samples): kan_hip_edge_linear_forward_workspace. */
int kan_hip_edge_linear_forward_supported(int dtype, int64_t n, int64_t in_features,
                                          int64_t out_features, int64_t num_basis);
int kan_hip_edge_linear_forward_workspace(int dtype, int64_t n, int64_t in_features,
                                          int64_t out_features, int64_t num_basis,
                                          size_t* bytes);
int kan_hip_edge_linear_forward(int dtype, const void* s, const void* basis,
                                const void* base_weight, const void* weight, void* y, void* a,
                                void* workspace, size_t workspace_bytes, int64_t n,
                                int64_t in_features, int64_t out_features, int64_t num_basis,
                                void* stream);

/* Double backward of the edge statistic, used when the regulariser's
 * backward is itself recorded (create_graph=True).  With the sign pattern
 * S = sign(phi) of the forward operands held fixed (its derivative is zero
 * almost everywhere), the first-order gradients ds, dH, dbw, dW of
 * kan_hip_edge_abs_mean_backward are linear in ga and in the operands they
 * contract; given incoming gradients u_ds [n, I], u_dH [n, I, R],
 * u_dbw [O, I], u_dW [O, I, R] (any may be NULL = zero) this writes
 *   g_ga[o,i]   = (1/n) sum_m S (u_ds bw + <u_dH, W> + s u_dbw + <H, u_dW>)
 *   g_bw, g_W   = (1/n) sum_m S ga [u_ds, u_dH]          (over samples)
 *   g_s, g_H    = (1/n) sum_o S ga [u_dbw, u_dW]         (over outputs)
 * (any output may be NULL).  Replaces the dense differentiable formulas of
 * EdgeAbsMean.backward under create_graph (spline_kan/fused.py:80-95),
 * which build the [n, O, I] sign tensor.  Workspace: query with the
 * _workspace call. */
int kan_hip_edge_abs_mean_double_backward_workspace(int dtype, int64_t n, int64_t in_features,
                                                    int64_t out_features, int64_t R,
                                                    size_t* bytes);
int kan_hip_edge_abs_mean_double_backward(int dtype, const void* grad_a, const void* s,
                                          const void* H, const void* base_weight, const void* W,
                                          const void* u_ds, const void* u_dH, const void* u_dbw,
                                          const void* u_dW, void* g_ga, void* g_s, void* g_H,
                                          void* g_bw, void* g_W, void* ws, size_t ws_bytes,
                                          int64_t n, int64_t in_features, int64_t out_features,
                                          int64_t R, void* stream);

/* Regulariser of one layer from its edge means a [count] (the KAN paper's
 * activation penalty):
 *   reg = mu1 * T + mu2 * H,   T = sum a,   H = -sum p log p,
 *   p = max(a / max(T, tiny), tiny)   (tiny = the type's smallest normal),
 * written to reg[0] (device).  Replaces regularization_from_edge_means
 * (spline_kan/reference_backend.py:149-170), an ATen expression of about
 * ten launches, with three; block sums in double, added in a fixed order.
 * The workspace (kan_hip_edge_reg_workspace bytes) keeps the statistics the
 * backward reads: pass the same one, unchanged, to
 * kan_hip_edge_reg_backward, which writes grad_a [count] =
 * grad_reg[0] * d reg / d a, with the clamps' zero-gradient masks (what
 * autograd takes through the reference expression). */
int kan_hip_edge_reg_workspace(int dtype, int64_t count, size_t* bytes);
int kan_hip_edge_reg(int dtype, const void* a, int64_t count, double mu1, double mu2, void* reg,
                     void* workspace, size_t workspace_bytes, void* stream);
int kan_hip_edge_reg_backward(int dtype, const void* grad_reg, const void* a, int64_t count,
                              double mu1, double mu2, const void* workspace,
                              size_t workspace_bytes, void* grad_a, void* stream);

/* Gram matrices of the least-squares spline refit used by update_grid and
 * extend_grid, per input feature i, accumulated in float64:
 *   gram[i]  = sum_b bn(x[b,i]) bn(x[b,i])^T   [I, Rn, Rn]  (A^T A on the new grid)
 *   cross[i] = sum_b bn(x[b,i]) bo(x[b,i])^T   [I, Rn, Ro]  (new basis x old basis)
 * with bn / bo the order-k bases on grid_new [I, G_new+2k+1] and grid_old
 * [I, G_old+2k+1] (Rn = G_new + k, Ro = G_old + k), and x_t the samples in
 * feature-major layout [I, n].  cross[i] times the old coefficients gives the
 * refit right-hand side A^T y_old, so this replaces the [O, B, I] curve
 * einsum and the normal-equation inputs of update_grid / curve2coeff and
 * extend_grid / fit_spline_coeffs (spline_kan/reference_backend.py:199-202,
 * 483-489; spline_kan/kan_linear.py:580-582).  Deterministic (fixed-order
 * sums, no atomics). */
int kan_hip_refit_gram(int dtype, const void* x_t, const void* grid_old, const void* grid_new,
                       double* gram, double* cross, int64_t n, int64_t in_features,
                       int64_t grid_size_old, int64_t grid_size_new, int64_t spline_order,
                       void* stream);

/* Kernel-level timing (measurement support; no counterpart in the
 * reference, whose benchmarks time with torch.profiler,
 * benchmarks/bench_kan.py:288-301).  kan_hip_timing_enable(1) clears the
 * record and starts recording a HIP-event pair around every kernel launch
 * the library makes, on the launch's own stream, together with the launch's
 * algorithmic work; kan_hip_timing_enable(0) clears and stops.
 * kan_hip_timing_read waits for the recorded events of one kernel class and
 * returns the summed duration (ms), the launch count and the summed work
 * (flops for class 0, bytes for classes 1-2, flops for classes 3-4).
 * Classes: 0 contraction GEMM, 1 basis, 2 basis_grad, 3 edge statistic,
 * 4 edge statistic backward, 5 packing/finalize, 6 streaming probe. */
int kan_hip_timing_enable(int on);
int kan_hip_timing_read(int kernel_class, double* total_ms, int64_t* launches, double* work);

/* Streaming probe (measurement support, no reference counterpart): float4
 * kernels that write a (mode 0), read a (mode 1; b receives nothing in
 * practice but must be a valid 4-byte buffer) or copy a to b (mode 2), over
 * `bytes` (a multiple of 16; 16-byte aligned buffers); mode 3 writes a in
 * the row-segment pattern of the basis kernel at c3's layout (whole rows of
 * 14336 floats that fit in `bytes`); modes 4 (write), 5 (read a, write
 * [rows, 1024] floats of b) and 6 (write) are candidate patterns on that
 * layout: one row segment per workgroup, and mode 3 with one step per
 * workgroup; 7 and 8 write 4 and 16 rows per workgroup, one whole-workgroup
 * segment at a time; 9 writes one segment per one-wave workgroup; 10 reads
 * two adjacent segments per workgroup (b as in mode 5).  Timed as kernel
 * class 6 with the bytes
 * moved as work; the HBM ceilings the memory-bound kernels are compared
 * with. */
int kan_hip_stream_probe(int mode, void* a, void* b, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KAN_HIP_H_ */

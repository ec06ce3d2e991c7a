/*
 * converse2d.h -- C ABI of the MI355X (gfx950) Converse2D forward library (libcvn_hip.so).
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream, enqueues its kernels on
 * that stream and returns without synchronising.  The caller owns all buffers; entry points that
 * need scratch memory take a caller-provided workspace whose size a matching *_workspace() query
 * returns (no entry point allocates device memory).  Entry points are re-entrant; the library's
 * mutable global state is the per-thread error string and, for cvn_converse2d_fwd_noalloc_f32 only,
 * a file-scope device array of CVN_NOALLOC_SCRATCH_BYTES (64 MiB) that the code object reserves on
 * every device of every process that loads the library, whether or not that entry point is called
 * (calls of that entry point that overlap on one device race on it).  Tensors are fp32, NCHW,
 * contiguous.  Return value: CVN_OK, or a negative CVN_ERR_* code with a message retrievable
 * through cvn_last_error() on the calling thread.
 *
 * Reference interfaces replaced (paths relative to the ConverseNet repository root):
 *   cvn_converse2d_op_f32   <- converse2d_forward (Converse2D/torch_converse2d/converse2d.cpp:165-209),
 *                              registered as converse2d::forward (converse2d.cpp:218-227); its table /
 *                              apply split mirrors the op's OTF cache (p2o_cached, converse2d.cpp:52-102)
 *   cvn_converse2d_fwd_f32  <- Converse2D.forward (models/util_converse.py:142-192): padding
 *                              (:144-145), x0 = nearest (:172-173), the solve (:175-187) and the crop
 *                              (:189-190) in one call; also ConvReverseDataNet.forward
 *                              (models/converse_usrnet.py:41-68) through psf_batch = B
 *   cvn_layernorm_cf_f32    <- LayerNorm(data_format="channels_first").forward (util_converse.py:63-68)
 *   cvn_conv1x1_f32         <- nn.Conv2d(cin, cout, 1, 1, 0) followed by nn.GELU() and/or a
 *                              residual add, as composed in ConverseBlock (util_converse.py:278-292)
 *                              and ConverseBlockAlphaVariant (util_converse.py:307-323)
 *   cvn_clear_cache         <- clear_fb_cache / converse2d::clear_cache (converse2d.cpp:211-216,221)
 */
#ifndef CONVERSE2D_H_
#define CONVERSE2D_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* cvn_stream_t; /* hipStream_t; NULL = default stream */

enum {
  CVN_OK = 0,
  CVN_ERR_ARG = -1,         /* bad shape / argument (the reference raises RuntimeError) */
  CVN_ERR_UNSUPPORTED = -2, /* valid for the reference but outside this library's limits */
  CVN_ERR_WORKSPACE = -3,   /* workspace missing or smaller than the *_workspace() query */
  CVN_ERR_HIP = -4          /* a HIP runtime call or kernel launch failed */
};

/* padding_mode of Converse2D (util_converse.py:112): F.pad modes */
enum { CVN_PAD_ZEROS = 0, CVN_PAD_REFLECT = 1, CVN_PAD_REPLICATE = 2, CVN_PAD_CIRCULAR = 3 };

/* activation applied to an output on store */
enum { CVN_ACT_NONE = 0, CVN_ACT_GELU = 1 };

const char* cvn_version(void);
const char* cvn_last_error(void);

/* Module-level fused forward.  x: (B,C,H,W).  psf: (psf_batch,C,kh,kw) with psf_batch 1 (shared,
 * Converse2D.weight) or B (per-sample, ConvReverseDataNet's k).  bias: (C) (Converse2D.bias or
 * ConvReverseDataNet.alpha), lambda = sigmoid(bias - 9) + eps.  The input is padded by `pad` on
 * every side with `pad_mode`, upsampled by `scale`, solved, and cropped back:
 * out: (B,C,H*scale,W*scale).  act = CVN_ACT_GELU applies exact GELU on store. */
size_t cvn_converse2d_fwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch,
                                    int kh, int kw, int scale, int pad);
int cvn_converse2d_fwd_f32(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                           const float* psf, int64_t psf_batch, int kh, int kw, const float* bias,
                           float eps, int scale, int pad, int pad_mode, int act, float* out,
                           void* workspace, size_t workspace_bytes, cvn_stream_t stream);

/* The module-level forward above without any allocation and without a caller workspace.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Its table and scratch live in a file-scope
 * device array of CVN_NOALLOC_SCRATCH_BYTES that each device holds until the process ends; a call whose
 * cvn_converse2d_fwd_workspace() exceeds it returns CVN_ERR_UNSUPPORTED (cfg1-cfg3-sized calls fit; a
 * Converse-DnCNN layer at B = 8 does not).  Calls on one device share the array: calls that overlap on
 * one device race. */
#define CVN_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int cvn_converse2d_fwd_noalloc_f32(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                                   const float* psf, int64_t psf_batch, int kh, int kw, const float* bias,
                                   float eps, int scale, int pad, int pad_mode, int act, float* out,
                                   cvn_stream_t stream);

/* Which kernels serve a module-level call, and so which layout its transfer table has:
 * CVN_ROUTE_FUSED    a plane per workgroup: padded planes of 132 x 132, 256 x 256 and 260 x 260 at
 *                    s = 1 (one kernel; two when scratch is given and there are at most 128 planes),
 *                    and upsampling onto 132 x 132 (s = 2-4) or 256 x 256 (s = 4, from 64 x 64)
 * CVN_ROUTE_PFA268   the three-pass 268 x 268 path (Converse-DnCNN's k7 p6 layers on 256 x 256 inputs)
 * CVN_ROUTE_GENERIC  the three-pass path for any plane up to 4096 x 4096, any scale, any psf size
 * CVN_ROUTE_AUTO     (argument only) the route cvn_converse2d_route() picks. */
enum { CVN_ROUTE_AUTO = 0, CVN_ROUTE_FUSED = 1, CVN_ROUTE_PFA268 = 2, CVN_ROUTE_GENERIC = 3 };

/* The route the library picks for a geometry (> 0), or a negative CVN_ERR_* code.  CVN_DISABLE_FUSED=1
 * in the environment makes it CVN_ROUTE_GENERIC; nothing else reads the environment when an explicit
 * route is passed below. */
int cvn_converse2d_route(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch, int kh, int kw, int scale,
                         int pad);

/* CVN_OK when the module-level forward (and, if asked, the backward for grad_x and / or the weight and
 * bias gradients) supports this geometry; otherwise CVN_ERR_UNSUPPORTED or CVN_ERR_ARG with the reason in
 * cvn_last_error().  Launches nothing.  The reference's PyTorch path has no such limits, so callers route
 * unsupported shapes to it (as util_converse.py:150-169 chooses between its backends). */
int cvn_converse2d_supported(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch, int kh, int kw,
                             int scale, int pad, int grad_x, int grad_weight);

/* The same forward in two steps, so that the transfer table (the psf's optical transfer function
 * combined with lambda into the closed-form solve, in the route's layout) can be cached across calls
 * while weight and bias are unchanged, as the reference caches its OTF (converse2d.cpp:52-102).
 * cvn_converse2d_table_f32 writes the table for a route; cvn_converse2d_apply_f32 runs that route with
 * it.  The caller keeps the route and the table's size with the table: the apply runs the route it is
 * given (CVN_ERR_ARG if that route does not serve the geometry, or if table_bytes is smaller than the
 * route's table), so a table is never read in a layout it was not written in.  The table depends on
 * (psf, psf_batch, bias, eps, C, H, W, scale, pad, route) and, for psf_batch = B, on B.
 * cvn_converse2d_fwd_f32 == table into workspace[0, align256(table_bytes)) + apply with the rest, on
 * the route cvn_converse2d_route() picks.  On CVN_ROUTE_FUSED the scratch may be null: with at most
 * 128 planes (B C) the route asks for scratch_bytes > 0 so that each plane's two row groups can run in
 * workgroups of their own (twice the CUs busy); given null, the apply runs one workgroup per plane.
 * On CVN_ROUTE_PFA268 the table must be 16-byte aligned (CVN_ERR_ARG otherwise). */
size_t cvn_converse2d_table_bytes(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch,
                                  int kh, int kw, int scale, int pad, int route);
size_t cvn_converse2d_scratch_bytes(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch,
                                    int kh, int kw, int scale, int pad, int route);
int cvn_converse2d_table_f32(const float* psf, int64_t psf_batch, int kh, int kw, const float* bias,
                             float eps, int64_t B, int64_t C, int64_t H, int64_t W, int scale, int pad,
                             int route, void* table, size_t table_bytes, cvn_stream_t stream);
int cvn_converse2d_apply_f32(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                             int64_t psf_batch, int kh, int kw, int scale, int pad, int pad_mode,
                             int act, int route, const void* table, size_t table_bytes, void* scratch,
                             size_t scratch_bytes, float* out, cvn_stream_t stream);

/* Backward of the module-level forward (act = none), the gradients the reference obtains by autograd
 * through Converse2D.forward (util_converse.py:142-192; its op is registered
 * CompositeImplicitAutograd, converse2d.cpp:223-227; gradient checks in test/test_error.py:51-54).
 * grad_out: (B,C,H*scale,W*scale).  Outputs (each may be null when not wanted): grad_x (B,C,H,W),
 * grad_psf (psf_batch,C,kh,kw), grad_bias (C).  x is read only for grad_psf / grad_bias.  Weight
 * gradients support scale <= 4.  The workspace may have any alignment: the query includes 256 bytes
 * of slack, and the regions are laid out from the first 256-byte boundary inside it. */
size_t cvn_converse2d_bwd_workspace(int64_t B, int64_t C, int64_t H, int64_t W, int64_t psf_batch,
                                    int kh, int kw, int scale, int pad);
int cvn_converse2d_bwd_f32(const float* grad_out, const float* x, int64_t B, int64_t C, int64_t H,
                           int64_t W, const float* psf, int64_t psf_batch, int kh, int kw,
                           const float* bias, float eps, int scale, int pad, int pad_mode,
                           float* grad_x, float* grad_psf, float* grad_bias, void* workspace,
                           size_t workspace_bytes, cvn_stream_t stream);

/* Op-level forward with the reference op's semantics: x (B,C,h,w) is the already padded input,
 * x0 (B,C,h*scale,w*scale) is arbitrary, psf (1,C,kh,kw), bias (C).  out: (B,C,h*scale,w*scale),
 * uncropped.  cvn_converse2d_op_f32 == cvn_converse2d_op_table_f32 into workspace[0, op_table_bytes)
 * + cvn_converse2d_op_apply_f32 with the rest.  The op table (FFT plan tables, the OTF and the alias-class
 * terms of the solve) depends on (psf, bias, eps, C, h, w, scale) only, not on B, x or x0: it is what the
 * reference's OTF cache keeps (p2o_cached, converse2d.cpp:58-102), and callers may cache it the same way. */
size_t cvn_converse2d_op_workspace(int64_t B, int64_t C, int64_t h, int64_t w, int kh, int kw,
                                   int scale);
int cvn_converse2d_op_f32(const float* x, const float* x0, int64_t B, int64_t C, int64_t h,
                          int64_t w, const float* psf, int kh, int kw, const float* bias,
                          float eps, int scale, float* out, void* workspace,
                          size_t workspace_bytes, cvn_stream_t stream);
/* Which kernels cvn_converse2d_op_apply_f32 runs for (h, w, scale) with 16-byte aligned x, x0 and out:
 * CVN_ROUTE_OP_PLANNED (scale 2-4, h in {64, 128, 256}, w and w * scale in {64, 128, 192, 256, 384, 512,
 * 768, 1024}: three passes on compile-time transform plans, one column block per mirrored pair of
 * alias classes) or CVN_ROUTE_GENERIC (runtime plans).  Both compute the same solve; misaligned
 * buffers always take the generic kernels.  No reference counterpart: converse2d.cpp:165-209 has one
 * code path. */
enum { CVN_ROUTE_OP_PLANNED = 4 };
int cvn_converse2d_op_route(int64_t h, int64_t w, int scale);
size_t cvn_converse2d_op_table_bytes(int64_t C, int64_t h, int64_t w, int kh, int kw, int scale);
size_t cvn_converse2d_op_scratch_bytes(int64_t B, int64_t C, int64_t h, int64_t w, int scale);
int cvn_converse2d_op_table_f32(const float* psf, int kh, int kw, const float* bias, float eps, int64_t C,
                                int64_t h, int64_t w, int scale, void* table, size_t table_bytes,
                                cvn_stream_t stream);
int cvn_converse2d_op_apply_f32(const float* x, const float* x0, int64_t B, int64_t C, int64_t h, int64_t w,
                                int scale, const void* table, size_t table_bytes, void* scratch,
                                size_t scratch_bytes, float* out, cvn_stream_t stream);

/* The reference keeps an OTF cache inside its op (converse2d.cpp:52-102).  This library keeps no cache:
 * transfer tables live in buffers the caller owns and may keep (the Python host caches them and
 * converse2d::clear_cache drops that cache).  This entry point has nothing to clear and returns CVN_OK;
 * it is kept so that a binding of the reference's clear_cache has a symbol to call. */
int cvn_clear_cache(void);

/* y = weight[c] * (x - mean_c) / sqrt(var_c + eps) + bias[c], statistics over C per pixel.
 * x, y: (B,C,HW). */
int cvn_layernorm_cf_f32(const float* x, int64_t B, int64_t C, int64_t HW, const float* weight,
                         const float* bias, float eps, float* y, cvn_stream_t stream);

/* y[b,o,p] = act(sum_c W[o,c] x[b,c,p] + bias[o]);  then, if residual != NULL,
 * y = (res_scale ? res_scale[o] : 1) * y + residual[b,o,p].  x: (B,Cin,HW), W: (Cout,Cin),
 * bias: (Cout) or NULL, residual: (B,Cout,HW) or NULL, res_scale: (Cout) or NULL.
 * y may alias residual.  Channel counts with a matrix-core tile run on the MFMA units: in whole
 * 32-channel chunks as split-fp16 products (each fp32 operand x = x_h + x_l, two fp16 parts; three
 * fp16 MFMAs accumulating in fp32; relative error per product below 2^-20, a chunk whose activations
 * leave fp16's range falls back to fp32 MFMAs), otherwise as fp32 MFMAs; 1 or 3 channels, and pixel
 * counts not a multiple of 4, run on a VALU kernel in fp32. */
int cvn_conv1x1_f32(const float* x, int64_t B, int64_t Cin, int64_t HW, const float* weight,
                    const float* bias, int64_t Cout, int act, const float* residual,
                    const float* res_scale, float* y, cvn_stream_t stream);

/* LayerNorm (channels_first) fused into the prologue of a 1x1 conv: the ConverseBlock front end
 * LN -> nn.Conv2d(cin, cout, 1) -> GELU (util_converse.py:278-280, 285-287).  Arguments as in
 * cvn_conv1x1_f32 plus the LayerNorm affine (Cin) and eps. */
int cvn_ln_conv1x1_f32(const float* x, int64_t B, int64_t Cin, int64_t HW, const float* ln_w,
                       const float* ln_b, float ln_eps, const float* weight, const float* bias,
                       int64_t Cout, int act, const float* residual, const float* res_scale,
                       float* y, cvn_stream_t stream);

/* The whole ConverseBlock conv2 branch with its residual (util_converse.py:285-288,292 and the
 * alpha-scaled form :314-317,322): y = x + res_scale * (W2 GELU(W1 LN(x) + b1) + b2).
 * x, y: (B,C,HW) (y may alias x), w1: (Cmid,C), w2: (C,Cmid), res_scale: (C) or NULL. */
int cvn_ln_mlp_residual_f32(const float* x, int64_t B, int64_t C, int64_t HW, const float* ln_w,
                            const float* ln_b, float ln_eps, const float* w1, const float* b1,
                            int64_t Cmid, const float* w2, const float* b2,
                            const float* res_scale, float* y, cvn_stream_t stream);

/* The ConverseBlock tail in one call (util_converse.py:279-293; alpha-scaled :309-323): the first
 * branch's last 1x1 and residual, y' = x + res_scale1 * (w0 a(t) + b0), then the conv2 branch,
 * y = y' + res_scale2 * (W2 GELU(W1 LN(y') + b1) + b2); y' never reaches memory.  t: (B,Ct,HW);
 * t_act = CVN_ACT_GELU: a(t) = GELU(t) (t is the Converse2D output, the block's GELU applied here
 * instead of on the Converse2D's store), CVN_ACT_NONE: a(t) = t (t already holds that GELU).
 * x, y: (B,C,HW) (y may alias x, not t), w0: (C,Ct),
 * w1: (Cmid,C), w2: (C,Cmid), res_scale1/2: (C) or NULL.  Instantiated for (Ct, C, Cmid) =
 * (128, 64, 128), the shape of Converse-DnCNN's and Converse-USRNet's blocks; other shapes return
 * CVN_ERR_UNSUPPORTED (use cvn_conv1x1_f32 + cvn_ln_mlp_residual_f32). */
int cvn_conv_ln_mlp_residual_f32(const float* t, int t_act, int64_t B, int64_t Ct, int64_t HW,
                                 const float* w0, const float* b0, const float* res_scale1, const float* x,
                                 int64_t C, const float* ln_w, const float* ln_b, float ln_eps,
                                 const float* w1, const float* b1, int64_t Cmid, const float* w2,
                                 const float* b2, const float* res_scale2, float* y, cvn_stream_t stream);
/* The same tail followed by the next block's first layer (util_converse.py:278-280, LN -> 1x1 -> GELU),
 * for chains of blocks (converse_dncnn.py:24, converse_usrnet.py:19-33): additionally
 * t_next = GELU(head_w LN_head(y) + head_b), (B,Ct,HW), head_w: (Ct,C).  t_next may alias
 * neither x nor y. */
int cvn_conv_ln_mlp_head_f32(const float* t, int t_act, int64_t B, int64_t Ct, int64_t HW,
                             const float* w0, const float* b0, const float* res_scale1, const float* x,
                             int64_t C, const float* ln_w, const float* ln_b, float ln_eps,
                             const float* w1, const float* b1, int64_t Cmid, const float* w2,
                             const float* b2, const float* res_scale2, float* y, const float* head_ln_w,
                             const float* head_ln_b, float head_ln_eps, const float* head_w,
                             const float* head_b, float* t_next, cvn_stream_t stream);

/* Plain device copy of n floats (bandwidth calibration). */
int cvn_copy_f32(const float* src, float* dst, int64_t n, cvn_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CONVERSE2D_H_ */

/* colabfold_gfx950_xla.h: the XLA FFI handler symbols of the gfx950 library.
 *
 * The same names the reference's libraries export through XLA_FFI_DEFINE_HANDLER_SYMBOL,
 * each with the reference's binding (context, arguments, results and attributes, in order) and
 * traits. A JAX caller registers them with
 *     jax.ffi.register_ffi_target(name, jax.ffi.pycapsule(fn), platform="ROCM")
 * Each decodes its call frame and calls the matching C entry point of colabfold_gfx950.h.
 * The XLA types are XLA's (xla/ffi/api/c_api.h); only pointers to them cross this interface.
 */
#ifndef COLABFOLD_GFX950_XLA_H_
#define COLABFOLD_GFX950_XLA_H_

#ifdef __cplusplus
extern "C" {
#endif

struct XLA_FFI_CallFrame;
struct XLA_FFI_Error;

/* cuda/volta_mma_attn.cu:625-640. ctx stream, device; args q, k, v, bias F16, kmask U8;
 * rets out F16, lse F32; attrs scale f32, block_q i64, block_k i64, want_lse bool.
 * Command-buffer compatible. */
struct XLA_FFI_Error* VoltaMma(struct XLA_FFI_CallFrame* call_frame);

/* volta_mma_attn.cu:594-607. args p, bias F16, kmask U8, gate_bias F16; ret out F16;
 * attrs scale, block_q, block_k, column bool. Command-buffer compatible. */
struct XLA_FFI_Error* VoltaMmaPacked(struct XLA_FFI_CallFrame* call_frame);

/* volta_mma_attn.cu:609-623. As VoltaMmaPacked with lims S32 after gate_bias. */
struct XLA_FFI_Error* VoltaMmaPackedTrim(struct XLA_FFI_CallFrame* call_frame);

/* cuda/volta_mma_attn_bwd.cu:455-473. ctx stream, device, scratch; args q, k, v, bias F16,
 * kmask U8, out, dout F16, lse F32; rets dq, dk, dv F16, dbias F32; attrs scale f32,
 * want_dbias bool. Not command-buffer compatible. */
struct XLA_FFI_Error* VoltaMmaBwd(struct XLA_FFI_CallFrame* call_frame);

/* cuda/volta_fused_ffi.h:337-351. args F16, F32, F32, F16, F16, F16, F16, F16; rets F16, F16;
 * attr eps. */
struct XLA_FFI_Error* VoltaLnGdp(struct XLA_FFI_CallFrame* call_frame);

/* volta_fused_ffi.h:353-371. args F32, F16, F32, F32, F32, F32, F16, F16, F16, F16, F16; ret F16;
 * attrs eps, add_input, has_keep. */
struct XLA_FFI_Error* VoltaTrimulEpilogue(struct XLA_FFI_CallFrame* call_frame);

/* volta_fused_ffi.h:373-388. args F16, F32, F32, F16, F16, F16; rets F16, F16;
 * attrs eps f32, n i64, heads i64, has_keep bool. */
struct XLA_FFI_Error* VoltaLnProj(struct XLA_FFI_CallFrame* call_frame);

/* volta_fused_ffi.h:390-401. args F16 x5; ret F16; attrs has_residual, has_keep. */
struct XLA_FFI_Error* VoltaOutProj(struct XLA_FFI_CallFrame* call_frame);

/* volta_fused_ffi.h:403-418. args F16, F32, F32, F16, F16, F16, F16, F16; ret F16;
 * attrs eps, add_input, has_keep. */
struct XLA_FFI_Error* VoltaTransition(struct XLA_FFI_CallFrame* call_frame);

/* cuda/volta_ops.cu:86-94. args x F16, scale F32, offset F32; ret F16; attr eps.
 * Command-buffer compatible. */
struct XLA_FFI_Error* VoltaLayerNorm(struct XLA_FFI_CallFrame* call_frame);

/* volta_ops.cu:258-269. ctx stream, device; args x, wp, bp, wg, bg, mask F16; ret F16;
 * attr activation i64. Command-buffer compatible. */
struct XLA_FFI_Error* VoltaGdp(struct XLA_FFI_CallFrame* call_frame);

/* cuda/volta_fused_ffi.h:420-431. ctx stream; args lhs, t F16, bias, norm F32, residual F16;
 * ret out F16; attrs eps f32, has_residual bool. Command-buffer compatible. */
struct XLA_FFI_Error* VoltaOpmUpdate(struct XLA_FFI_CallFrame* call_frame);

/* volta_fused_ffi.h:433-440. ctx stream; args left, right, wT F16; ret out F16.
 * Command-buffer compatible. */
struct XLA_FFI_Error* VoltaOpmOuter(struct XLA_FFI_CallFrame* call_frame);

#ifdef __cplusplus
}
#endif

#endif /* COLABFOLD_GFX950_XLA_H_ */

/* colabfold_gfx950.h: the C ABI of the gfx950 (MI355X) ColabFold legacy-kernel library.
 *
 * One entry point per XLA FFI target of the reference. Each takes the stream, the buffers in
 * the FFI binding's order (arguments, then results) and the FFI attributes, and returns a
 * status: CLK_OK, CLK_INVALID_ARGUMENT or CLK_INTERNAL (the XLA FFI / absl error codes). The
 * message of the last failure on the calling thread is clk_last_error(). Validation runs
 * before any HIP call, so a rejected call touches no device; work is enqueued on `stream`
 * only, with no host synchronisation. No entry point allocates device memory: the backward
 * takes its scratch as a workspace argument, as the reference takes it from XLA's
 * ScratchAllocator.
 *
 * Buffers are described by clk_buffer: a device pointer, an element type (the XLA FFI
 * DataType numbering), a rank and the dimensions, exactly what an XLA_FFI_Buffer carries.
 * Optional inputs and results follow the reference: a one-element buffer plus a flag
 * (want_lse, has_keep, has_residual, n == 0, heads == 0).
 */
#ifndef COLABFOLD_GFX950_H_
#define COLABFOLD_GFX950_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* clk_stream; /* a hipStream_t; NULL is the null stream */

enum clk_dtype { CLK_S32 = 4, CLK_U8 = 6, CLK_F16 = 10, CLK_F32 = 11, CLK_BF16 = 16 };

enum clk_status { CLK_OK = 0, CLK_INVALID_ARGUMENT = 3, CLK_INTERNAL = 13 };

typedef struct clk_buffer {
    void* data;
    int32_t dtype;       /* enum clk_dtype */
    int32_t rank;
    const int64_t* dims; /* rank entries, row-major, last dimension contiguous */
} clk_buffer;

/* The message of the last failed call on this thread ("" after a success). */
const char* clk_last_error(void);

/* Version of this library, e.g. "0.6.0+gfx950". */
const char* clk_version(void);

/* Measurement hook, no counterpart in the reference. With count > 0, each later entry point
 * records events[0] on its stream before its first kernel launch and events[i] after its i-th,
 * for i < count (hipEvent_t handles, owned by the caller). count 0 turns it off. The setting is
 * process-wide and meant for a single-threaded benchmark. */
int clk_set_stage_events(void* const* events, int32_t count);

/* ---- attention ------------------------------------------------------------------------ */

/* VoltaMma (reference cuda/volta_mma_attn.cu:522-542, handler 625-640).
 * q [N,H,Sq,D], k, v [N,H,Sk,D], bias [H,Sq,Sk] F16; kmask [N,Sk] U8
 * -> out [N,H,Sq,D] F16, lse [N,H,Sq] F32 (log2 domain; untouched, any size, without want_lse).
 * (D, block_q, block_k) must be one of the reference's dispatch entries (volta_mma_attn.cu:508-517). */
int clk_attention_fwd(clk_stream stream, int32_t device, const clk_buffer* q, const clk_buffer* k,
                      const clk_buffer* v, const clk_buffer* bias, const clk_buffer* kmask,
                      const clk_buffer* out, const clk_buffer* lse, float scale, int64_t block_q,
                      int64_t block_k, int32_t want_lse);

/* VoltaMmaPacked (volta_mma_attn.cu:544-583, handler 594-607): q, k, v (and the gate when
 * G == 4) read in place from p [X,Y,G,H,D]; out [X,Y,H,D]; rows attend along Y, columns
 * (column != 0) along X. bias [H,S,S], kmask [N,S], gate_bias [H,D] (any size when G == 3). */
int clk_attention_packed(clk_stream stream, int32_t device, const clk_buffer* p,
                         const clk_buffer* bias, const clk_buffer* kmask,
                         const clk_buffer* gate_bias, const clk_buffer* out, float scale,
                         int64_t block_q, int64_t block_k, int32_t column);

/* VoltaMmaPackedTrim (volta_mma_attn.cu:585-592, handler 609-623): as clk_attention_packed
 * with lims S32 [N+1] (each batch row's last live key + 1, then the largest). */
int clk_attention_packed_trim(clk_stream stream, int32_t device, const clk_buffer* p,
                              const clk_buffer* bias, const clk_buffer* kmask,
                              const clk_buffer* gate_bias, const clk_buffer* lims,
                              const clk_buffer* out, float scale, int64_t block_q,
                              int64_t block_k, int32_t column);

/* VoltaMmaBwd (reference cuda/volta_mma_attn_bwd.cu:385-451, handler 455-473).
 * q, k, v, bias F16; kmask U8; out, dout F16; lse F32 [N,H,Sq] -> dq, dk, dv F16,
 * dbias F32 [H,Sq,Sk] (the sum of dS over the N rows; all zeros without want_dbias).
 * workspace: device scratch of at least clk_attention_bwd_workspace_size() bytes, 256-byte
 * aligned; the reference takes the same kind of scratch from XLA's ScratchAllocator.
 * Results are bit-identical from run to run (no atomics). */
int clk_attention_bwd(clk_stream stream, int32_t device, const clk_buffer* q, const clk_buffer* k,
                      const clk_buffer* v, const clk_buffer* bias, const clk_buffer* kmask,
                      const clk_buffer* out, const clk_buffer* dout, const clk_buffer* lse,
                      const clk_buffer* dq, const clk_buffer* dk, const clk_buffer* dv,
                      const clk_buffer* dbias, float scale, int32_t want_dbias, void* workspace,
                      size_t workspace_bytes);

/* Bytes of workspace clk_attention_bwd needs for these shapes on this device (0 on a shape the
 * backward would reject; the call itself then reports why). */
size_t clk_attention_bwd_workspace_size(int32_t device, const clk_buffer* q, const clk_buffer* k);

/* No counterpart in the reference: clk_attention_bwd for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same buffers, flags,
 * validation and results (bit-identical), but no workspace argument: the scratch is a static
 * device array of the library, one per GPU, of clk_attention_bwd_noalloc_scratch_size() bytes
 * (96 MiB, enough for [512, 8, 384, 32]), held until the process ends. The array is part of the
 * library's code object, so loading the library reserves those 96 MiB on every GPU it runs a
 * kernel on, whether or not this entry point is ever called. Shapes whose scratch
 * would exceed it are rejected with CLK_INVALID_ARGUMENT before any launch. The call allocates
 * nothing. Every call on a GPU shares that GPU's scratch, so calls that overlap on one GPU (two
 * streams, or two threads) race and must be serialised by the caller. */
int clk_attention_bwd_noalloc(clk_stream stream, int32_t device, const clk_buffer* q,
                              const clk_buffer* k, const clk_buffer* v, const clk_buffer* bias,
                              const clk_buffer* kmask, const clk_buffer* out,
                              const clk_buffer* dout, const clk_buffer* lse, const clk_buffer* dq,
                              const clk_buffer* dk, const clk_buffer* dv, const clk_buffer* dbias,
                              float scale, int32_t want_dbias);

/* Bytes of the static scratch behind clk_attention_bwd_noalloc. */
size_t clk_attention_bwd_noalloc_scratch_size(void);

/* Diagnostic, no counterpart in the reference: the backward's launch plan for these shapes on
 * this device, plan[0..count) = {row groups per dK/dV workgroup, batch rows per workgroup
 * (chunk), chunks, row passes per workgroup, query windows, 1 where the dK/dV kernel keeps its
 * dBias partial in registers (D <= 32, Sq <= 384) else 0}. */
int clk_attention_bwd_plan(int32_t device, int64_t N, int64_t H, int64_t Sq, int64_t Sk,
                           int64_t D, int64_t* plan, int32_t count);

/* ---- LayerNorm-fused pair-stack projections (reference cuda/volta_fused_ffi.h) --------- */

/* Activation types, an addition to the reference (whose handlers bind F16 only): the activation
 * buffers of each entry point below (x, o, residual and every activation result: left, right,
 * out, p, bias) may be BF16 instead of F16, all together; weights, biases and keep stay F16 and
 * LayerNorm parameters F32. A BF16 input is read exactly into fp32, the LayerNorm output (and
 * o, and the transition's hidden activation) enter the matrix cores as fp16, and the results
 * are rounded to BF16 once. A mix of F16 and BF16 activations is CLK_INVALID_ARGUMENT. The XLA
 * FFI handlers keep the reference's F16-only binding. */

/* VoltaLnGdp (volta_fused_ffi.h:42-80, handler 337-351): left, right [P/2, M] = the two halves
 * of max(mask,0) * (y@wp + bp) * sigmoid(y@wg + bg), channel major, y = LN(x).
 * x [M,K] F16; scale, offset [K] F32; wpT [P,K], bp [P], wgT [P,K], bg [P], mask [M] F16.
 * K and P/2 in {64, 128}. The mask is also the row-tile keep. */
int clk_ln_gdp(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
               const clk_buffer* offset, const clk_buffer* wpT, const clk_buffer* bp,
               const clk_buffer* wgT, const clk_buffer* bg, const clk_buffer* mask,
               const clk_buffer* left, const clk_buffer* right, float eps);

/* VoltaTrimulEpilogue (volta_fused_ffi.h:82-133, handler 353-371):
 * out [M,O] = (LN(x_cm.T)@wo + bo) * sigmoid(LN_in(x)@wg + bg) [+ x with add_input].
 * x_cm [C,M] F32; x [M,CA] F16; in_scale, in_offset [CA], ln_scale, ln_offset [C] F32;
 * woT [O,C], bo [O], wgT [O,CA], bg [O], keep [M] (or any size without has_keep) F16.
 * C, CA, O in {64, 128}; O == CA with add_input (then out may alias x). */
int clk_trimul_epilogue(clk_stream stream, const clk_buffer* x_cm, const clk_buffer* x,
                        const clk_buffer* in_scale, const clk_buffer* in_offset,
                        const clk_buffer* ln_scale, const clk_buffer* ln_offset,
                        const clk_buffer* woT, const clk_buffer* bo, const clk_buffer* wgT,
                        const clk_buffer* bg, const clk_buffer* keep, const clk_buffer* out,
                        float eps, int32_t add_input, int32_t has_keep);

/* VoltaLnProj (volta_fused_ffi.h:135-176, handler 373-388): p [M,n] = LN(x)@w and
 * bias [heads,M] = (LN(x)@wb).T. x [M,K] F16 (K in {64,128}); scale, offset [K] F32;
 * wT [n,K], wbT [heads,K], keep [M] F16. n a multiple of 64 (0: p untouched), heads <= 8
 * (0: bias untouched). */
int clk_ln_projection(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
                      const clk_buffer* offset, const clk_buffer* wT, const clk_buffer* wbT,
                      const clk_buffer* keep, const clk_buffer* p, const clk_buffer* bias,
                      float eps, int64_t n, int64_t heads, int32_t has_keep);

/* VoltaOutProj (volta_fused_ffi.h:178-214, handler 390-401): out [M,N] = o@w + b
 * [+ residual]. o [M,K], wT [N,K], b [N], residual [M,N], keep [M] F16; K, N in {64,128}.
 * With has_residual out may alias residual. */
int clk_output_projection(clk_stream stream, const clk_buffer* o, const clk_buffer* wT,
                          const clk_buffer* b, const clk_buffer* residual, const clk_buffer* keep,
                          const clk_buffer* out, int32_t has_residual, int32_t has_keep);

/* VoltaTransition (volta_fused_ffi.h:216-259, handler 403-418): out [M,C] =
 * relu(LN(x)@w1 + b1)@w2 + b2 [+ x]. x [M,C] F16 (C in {64,128,256}); scale, offset [C] F32;
 * w1T [H,C], b1 [H], w2T [H/64][C][64] (w2T[j][c][i] = w2[64j+i][c]), b2 [C], keep [M] F16;
 * H in {2C, 4C}. With add_input out may alias x. */
int clk_transition(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
                   const clk_buffer* offset, const clk_buffer* w1T, const clk_buffer* b1,
                   const clk_buffer* w2T, const clk_buffer* b2, const clk_buffer* keep,
                   const clk_buffer* out, float eps, int32_t add_input, int32_t has_keep);

/* ---- unfused pair-stack ops (reference cuda/volta_ops.cu) ------------------------------ */

/* VoltaLayerNorm (volta_ops.cu:27-84, handler 86-94): out [M,C] = LN(x) over the last axis with
 * one-pass fp32 statistics (var = max(E[x^2] - mean^2, 0)). x [M,C] F16; scale, offset [C] F32;
 * out [M,C] F16. */
int clk_layer_norm(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
                   const clk_buffer* offset, const clk_buffer* out, float eps);

/* VoltaGdp (volta_ops.cu:97-256, handler 258-269): out [M,N] = mask * (x@wp + bp) *
 * act(x@wg + bg), act = sigmoid (activation 0) or swish (1). x [M,K]; wp, wg [K,N] row-major;
 * bp, bg [N]; mask [M]; all F16. N a multiple of 8. */
int clk_gated_dual_proj(clk_stream stream, int32_t device, const clk_buffer* x,
                        const clk_buffer* wp, const clk_buffer* bp, const clk_buffer* wg,
                        const clk_buffer* bg, const clk_buffer* mask, const clk_buffer* out,
                        int64_t activation);

/* ---- outer product mean (reference cuda/volta_ops.cu) ---------------------------------- */

/* VoltaOpmUpdate (volta_ops.cu:643-704, handler cuda/volta_fused_ffi.h:261-297, 420-431):
 * out[b,d,:] = fp16((lhs[b] @ t[:,d,:] + bias) / (eps + norm[b,d]) [+ residual[b,d,:]]), fp32
 * accumulation. lhs [B,K], t [K,D,F], residual [B,D,F] F16 (read only with has_residual; may
 * alias out); bias [F], norm [B,D] F32; out [B,D,F] F16. K a multiple of 32, F in
 * {16,32,64,128}, D at most 65535. */
int clk_opm_update(clk_stream stream, const clk_buffer* lhs, const clk_buffer* t,
                   const clk_buffer* bias, const clk_buffer* norm, const clk_buffer* residual,
                   const clk_buffer* out, float eps, int32_t has_residual);

/* VoltaOpmOuter (volta_ops.cu:706-792, handler volta_fused_ffi.h:299-335, 433-440):
 * out[b,d,f] = fp16(sum_c sum_e fp16(sum_a left[a,b,c] right[a,d,e]) wT[f, c E + e]) over the
 * 16 rows a. left [16,B,C], right [16,D,E=32], wT [F,C*E], out [B,D,F], all F16. C a multiple of
 * 16, D a multiple of 4 (D/4 at most 65535), F in {16,32,64,128}. */
int clk_opm_outer(clk_stream stream, const clk_buffer* left, const clk_buffer* right,
                  const clk_buffer* wT, const clk_buffer* out);

#ifdef __cplusplus
}
#endif

#endif /* COLABFOLD_GFX950_H_ */

// XLA FFI handler symbols of the reference's targets on this path, over the library's C ABI.
//
// Each exported `XLA_FFI_Error* Name(XLA_FFI_CallFrame*)` decodes the call frame the way the
// reference's XLA_FFI_DEFINE_HANDLER_SYMBOL bindings declare it (context, arguments, results and
// attributes in the orders of cuda/volta_mma_attn.cu:594-640, cuda/volta_mma_attn_bwd.cu:455-473,
// cuda/volta_fused_ffi.h:337-418 and cuda/volta_ops.cu:86-94, 258-269) and calls the matching clk_* entry point on the stream XLA
// provides. It answers XLA's metadata query with API version 0.1 and the reference's traits:
// every target is command-buffer compatible except VoltaMmaBwd. The backward's workspace comes
// from XLA's device allocator for the duration of the call, as the reference's ScratchAllocator
// scratch does (volta_mma_attn_bwd.cu:346-361). Failures return an XLA_FFI_Error carrying the
// C ABI's status (INVALID_ARGUMENT or INTERNAL) and message.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "colabfold_gfx950.h"
#include "colabfold_gfx950_xla.h"
#include "xla_ffi_api.h"

namespace {

constexpr uint32_t kCmdBuffer = CLK_XLA_FFI_TRAIT_COMMAND_BUFFER_COMPATIBLE;

class Frame {
   public:
    explicit Frame(XLA_FFI_CallFrame* cf) : cf_(cf) {}

    XLA_FFI_Error* error(XLA_FFI_Error_Code code, const std::string& msg) const {
        XLA_FFI_Error_Create_Args a;
        std::memset(&a, 0, sizeof(a));
        a.struct_size = sizeof(a);
        a.message = msg.c_str();
        a.errc = code;
        return cf_->api->XLA_FFI_Error_Create(&a);
    }
    XLA_FFI_Error* invalid(const std::string& msg) const {
        return error(XLA_FFI_Error_Code_INVALID_ARGUMENT, msg);
    }
    XLA_FFI_Error* status(int st) const {
        if (st == CLK_OK) return nullptr;
        return error(st == CLK_INVALID_ARGUMENT ? XLA_FFI_Error_Code_INVALID_ARGUMENT
                                                : XLA_FFI_Error_Code_INTERNAL,
                     clk_last_error());
    }

    // arguments then results, as clk_buffers; false (with why_) on a count or kind mismatch
    bool buffers(int64_t nargs, int64_t nrets, clk_buffer* out) {
        if (cf_->args.size != nargs) {
            why_ = "Wrong number of arguments: expected " + std::to_string(nargs) + " but got " +
                   std::to_string(cf_->args.size);
            return false;
        }
        if (cf_->rets.size != nrets) {
            why_ = "Wrong number of results: expected " + std::to_string(nrets) + " but got " +
                   std::to_string(cf_->rets.size);
            return false;
        }
        for (int64_t i = 0; i < nargs + nrets; ++i) {
            const bool arg = i < nargs;
            const int64_t j = arg ? i : i - nargs;
            const int kind = arg ? (int)cf_->args.types[j] : (int)cf_->rets.types[j];
            if (kind != 1) {
                why_ = std::string(arg ? "argument " : "result ") + std::to_string(j) + " is not a buffer";
                return false;
            }
            const XLA_FFI_Buffer* b =
                static_cast<const XLA_FFI_Buffer*>(arg ? cf_->args.args[j] : cf_->rets.rets[j]);
            out[i].data = b->data;
            out[i].dtype = (int32_t)b->dtype;
            out[i].rank = (int32_t)b->rank;
            out[i].dims = b->dims;
        }
        return true;
    }

    bool f32(const char* name, float* v) {
        const XLA_FFI_Scalar* s = scalar(name, XLA_FFI_DataType_F32, "f32");
        if (s != nullptr) *v = *static_cast<const float*>(s->value);
        return s != nullptr;
    }
    bool i64(const char* name, int64_t* v) {
        const XLA_FFI_Scalar* s = scalar(name, XLA_FFI_DataType_S64, "i64");
        if (s != nullptr) *v = *static_cast<const int64_t*>(s->value);
        return s != nullptr;
    }
    bool flag(const char* name, int32_t* v) {
        const XLA_FFI_Scalar* s = scalar(name, XLA_FFI_DataType_PRED, "bool");
        if (s != nullptr) *v = *static_cast<const uint8_t*>(s->value) != 0;
        return s != nullptr;
    }

    XLA_FFI_Error* decode_error() const { return invalid(why_); }

    bool stream(clk_stream* s) {
        XLA_FFI_Stream_Get_Args a;
        std::memset(&a, 0, sizeof(a));
        a.struct_size = sizeof(a);
        a.ctx = cf_->ctx;
        if (XLA_FFI_Error* e = cf_->api->XLA_FFI_Stream_Get(&a)) {
            pending_ = e;
            return false;
        }
        *s = static_cast<clk_stream>(a.stream);
        return true;
    }
    XLA_FFI_Error* pending() const { return pending_; }

    // the device the stream belongs to (the current device for the null stream)
    static int32_t device_of(clk_stream s) {
        int dev = -1;
        if (hipStreamGetDevice(reinterpret_cast<hipStream_t>(s), &dev) != hipSuccess) {
            (void)hipGetLastError();
            if (hipGetDevice(&dev) != hipSuccess) {
                (void)hipGetLastError();
                dev = -1;
            }
        }
        return dev;
    }

    void* allocate(size_t bytes, size_t alignment) {
        XLA_FFI_DeviceMemory_Allocate_Args a;
        std::memset(&a, 0, sizeof(a));
        a.struct_size = sizeof(a);
        a.ctx = cf_->ctx;
        a.size = bytes;
        a.alignment = alignment;
        if (XLA_FFI_Error* e = cf_->api->XLA_FFI_DeviceMemory_Allocate(&a)) {
            pending_ = e;
            return nullptr;
        }
        return a.data;
    }
    void release(void* data, size_t bytes) {
        XLA_FFI_DeviceMemory_Free_Args a;
        std::memset(&a, 0, sizeof(a));
        a.struct_size = sizeof(a);
        a.ctx = cf_->ctx;
        a.size = bytes;
        a.data = data;
        (void)cf_->api->XLA_FFI_DeviceMemory_Free(&a);  // XLA owns a failure to free
    }

   private:
    const XLA_FFI_Scalar* scalar(const char* name, XLA_FFI_DataType dtype, const char* tname) {
        const size_t len = std::strlen(name);
        for (int64_t i = 0; i < cf_->attrs.size; ++i) {
            const XLA_FFI_ByteSpan* n = cf_->attrs.names[i];
            if (n->len != len || std::memcmp(n->ptr, name, len) != 0) continue;
            const XLA_FFI_Scalar* s = static_cast<const XLA_FFI_Scalar*>(cf_->attrs.attrs[i]);
            if (cf_->attrs.types[i] != XLA_FFI_AttrType_SCALAR || s->dtype != dtype) {
                why_ = std::string("attribute ") + name + " must be a " + tname + " scalar";
                return nullptr;
            }
            return s;
        }
        why_ = std::string("missing attribute ") + name;
        return nullptr;
    }

    XLA_FFI_CallFrame* cf_;
    std::string why_;
    XLA_FFI_Error* pending_ = nullptr;
};

// True when the frame is XLA's metadata query (answered here with the API version and the
// traits) or a stage other than EXECUTE (nothing to do); false when the handler body should run.
bool preamble(XLA_FFI_CallFrame* cf, uint32_t traits) {
    for (XLA_FFI_Extension_Base* e = cf->extension_start; e != nullptr; e = e->next) {
        if (e->type == XLA_FFI_Extension_Metadata) {
            XLA_FFI_Metadata* m = reinterpret_cast<XLA_FFI_Metadata_Extension*>(e)->metadata;
            m->api_version.struct_size = sizeof(XLA_FFI_Api_Version);
            m->api_version.extension_start = nullptr;
            m->api_version.major_version = CLK_XLA_FFI_API_MAJOR;
            m->api_version.minor_version = CLK_XLA_FFI_API_MINOR;
            m->traits = traits;
            return true;
        }
    }
    return cf->stage != XLA_FFI_ExecutionStage_EXECUTE;
}

}  // namespace

extern "C" {

XLA_FFI_Error* VoltaMma(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[7];
    float scale;
    int64_t bq, bk;
    int32_t want_lse;
    if (!f.buffers(5, 2, b) || !f.f32("scale", &scale) || !f.i64("block_q", &bq) ||
        !f.i64("block_k", &bk) || !f.flag("want_lse", &want_lse)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_attention_fwd(s, Frame::device_of(s), &b[0], &b[1], &b[2], &b[3], &b[4],
                                      &b[5], &b[6], scale, bq, bk, want_lse));
}

static XLA_FFI_Error* packed(XLA_FFI_CallFrame* cf, bool trim) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[6];
    float scale;
    int64_t bq, bk;
    int32_t column;
    const int nargs = trim ? 5 : 4;
    if (!f.buffers(nargs, 1, b) || !f.f32("scale", &scale) || !f.i64("block_q", &bq) ||
        !f.i64("block_k", &bk) || !f.flag("column", &column)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    const int32_t dev = Frame::device_of(s);
    if (trim) {
        return f.status(clk_attention_packed_trim(s, dev, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5],
                                                  scale, bq, bk, column));
    }
    return f.status(clk_attention_packed(s, dev, &b[0], &b[1], &b[2], &b[3], &b[4], scale, bq, bk,
                                         column));
}

XLA_FFI_Error* VoltaMmaPacked(XLA_FFI_CallFrame* cf) { return packed(cf, false); }
XLA_FFI_Error* VoltaMmaPackedTrim(XLA_FFI_CallFrame* cf) { return packed(cf, true); }

XLA_FFI_Error* VoltaMmaBwd(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, 0u)) return nullptr;
    Frame f(cf);
    clk_buffer b[12];
    float scale;
    int32_t want_dbias;
    if (!f.buffers(8, 4, b) || !f.f32("scale", &scale) || !f.flag("want_dbias", &want_dbias)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    const int32_t dev = Frame::device_of(s);
    const size_t bytes = clk_attention_bwd_workspace_size(dev, &b[0], &b[1]);
    void* ws = nullptr;
    if (bytes > 0) {
        ws = f.allocate(bytes, 256);
        if (ws == nullptr) {
            if (f.pending() != nullptr) return f.pending();
            return f.error(XLA_FFI_Error_Code_INTERNAL, "volta_mma_bwd: no scratch for the workspace");
        }
    }
    const int st = clk_attention_bwd(s, dev, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5], &b[6], &b[7],
                                     &b[8], &b[9], &b[10], &b[11], scale, want_dbias, ws, bytes);
    if (ws != nullptr) f.release(ws, bytes);
    return f.status(st);
}

XLA_FFI_Error* VoltaLnGdp(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[10];
    float eps;
    if (!f.buffers(8, 2, b) || !f.f32("eps", &eps)) return f.decode_error();
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_ln_gdp(s, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5], &b[6], &b[7], &b[8],
                               &b[9], eps));
}

XLA_FFI_Error* VoltaTrimulEpilogue(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[12];
    float eps;
    int32_t add_input, has_keep;
    if (!f.buffers(11, 1, b) || !f.f32("eps", &eps) || !f.flag("add_input", &add_input) ||
        !f.flag("has_keep", &has_keep)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_trimul_epilogue(s, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5], &b[6], &b[7],
                                        &b[8], &b[9], &b[10], &b[11], eps, add_input, has_keep));
}

XLA_FFI_Error* VoltaLnProj(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[8];
    float eps;
    int64_t n, heads;
    int32_t has_keep;
    if (!f.buffers(6, 2, b) || !f.f32("eps", &eps) || !f.i64("n", &n) || !f.i64("heads", &heads) ||
        !f.flag("has_keep", &has_keep)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_ln_projection(s, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5], &b[6], &b[7], eps,
                                      n, heads, has_keep));
}

XLA_FFI_Error* VoltaOutProj(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[6];
    int32_t has_residual, has_keep;
    if (!f.buffers(5, 1, b) || !f.flag("has_residual", &has_residual) || !f.flag("has_keep", &has_keep)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_output_projection(s, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5], has_residual,
                                          has_keep));
}

XLA_FFI_Error* VoltaTransition(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[9];
    float eps;
    int32_t add_input, has_keep;
    if (!f.buffers(8, 1, b) || !f.f32("eps", &eps) || !f.flag("add_input", &add_input) ||
        !f.flag("has_keep", &has_keep)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_transition(s, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5], &b[6], &b[7], &b[8],
                                   eps, add_input, has_keep));
}

XLA_FFI_Error* VoltaLayerNorm(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[4];
    float eps;
    if (!f.buffers(3, 1, b) || !f.f32("eps", &eps)) return f.decode_error();
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_layer_norm(s, &b[0], &b[1], &b[2], &b[3], eps));
}

XLA_FFI_Error* VoltaGdp(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[7];
    int64_t activation;
    if (!f.buffers(6, 1, b) || !f.i64("activation", &activation)) return f.decode_error();
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_gated_dual_proj(s, Frame::device_of(s), &b[0], &b[1], &b[2], &b[3], &b[4],
                                        &b[5], &b[6], activation));
}

XLA_FFI_Error* VoltaOpmUpdate(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[6];
    float eps;
    int32_t has_residual;
    if (!f.buffers(5, 1, b) || !f.f32("eps", &eps) || !f.flag("has_residual", &has_residual)) {
        return f.decode_error();
    }
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_opm_update(s, &b[0], &b[1], &b[2], &b[3], &b[4], &b[5], eps, has_residual));
}

XLA_FFI_Error* VoltaOpmOuter(XLA_FFI_CallFrame* cf) {
    if (preamble(cf, kCmdBuffer)) return nullptr;
    Frame f(cf);
    clk_buffer b[4];
    if (!f.buffers(3, 1, b)) return f.decode_error();
    clk_stream s;
    if (!f.stream(&s)) return f.pending();
    return f.status(clk_opm_outer(s, &b[0], &b[1], &b[2], &b[3]));
}

}  // extern "C"

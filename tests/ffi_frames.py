"""ctypes model of the XLA FFI call frame (xla/ffi/api/c_api.h, API 0.1) and a mock of the XLA
API table, to drive the library's handler symbols without jax: the mock records the errors a
handler creates, hands out a stream and serves device-memory requests. Test infrastructure."""
import ctypes as C

PRED, S32, S64, U8, F16, F32 = 1, 4, 5, 6, 10, 11
INVALID_ARGUMENT, INTERNAL = 3, 13
EXECUTE = 3
ATTR_SCALAR = 3
BUFFER = 1
METADATA = 1


class ExtBase(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("type", C.c_int), ("next", C.c_void_p)]


class ApiVersion(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p),
                ("major_version", C.c_int), ("minor_version", C.c_int)]


class ErrorCreateArgs(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p),
                ("message", C.c_char_p), ("errc", C.c_int)]


class StreamGetArgs(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p), ("ctx", C.c_void_p),
                ("stream", C.c_void_p)]


class AllocArgs(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p), ("ctx", C.c_void_p),
                ("size", C.c_size_t), ("alignment", C.c_size_t), ("data", C.c_void_p)]


class FreeArgs(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p), ("ctx", C.c_void_p),
                ("size", C.c_size_t), ("data", C.c_void_p)]


ERROR_CREATE = C.CFUNCTYPE(C.c_void_p, C.POINTER(ErrorCreateArgs))
STREAM_GET = C.CFUNCTYPE(C.c_void_p, C.POINTER(StreamGetArgs))
ALLOCATE = C.CFUNCTYPE(C.c_void_p, C.POINTER(AllocArgs))
FREE = C.CFUNCTYPE(C.c_void_p, C.POINTER(FreeArgs))


class Api(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p),
                ("api_version", ApiVersion), ("internal_api", C.c_void_p),
                ("error_create", ERROR_CREATE), ("error_get_message", C.c_void_p),
                ("error_destroy", C.c_void_p), ("handler_register", C.c_void_p),
                ("stream_get", STREAM_GET), ("type_id_register", C.c_void_p),
                ("execution_context_get", C.c_void_p), ("state_set", C.c_void_p),
                ("state_get", C.c_void_p), ("device_memory_allocate", ALLOCATE),
                ("device_memory_free", FREE)]


class Buffer(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p), ("dtype", C.c_int),
                ("data", C.c_void_p), ("rank", C.c_int64), ("dims", C.POINTER(C.c_int64))]


class Args(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p), ("size", C.c_int64),
                ("types", C.POINTER(C.c_int)), ("args", C.POINTER(C.c_void_p))]


class ByteSpan(C.Structure):
    _fields_ = [("ptr", C.c_char_p), ("len", C.c_size_t)]


class Scalar(C.Structure):
    _fields_ = [("dtype", C.c_int), ("value", C.c_void_p)]


class Attrs(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p), ("size", C.c_int64),
                ("types", C.POINTER(C.c_int)), ("names", C.POINTER(C.POINTER(ByteSpan))),
                ("attrs", C.POINTER(C.c_void_p))]


class CallFrame(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("extension_start", C.c_void_p),
                ("api", C.POINTER(Api)), ("ctx", C.c_void_p), ("stage", C.c_int), ("args", Args),
                ("rets", Args), ("attrs", Attrs)]


class Metadata(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("api_version", ApiVersion), ("traits", C.c_uint32)]


class MetadataExtension(C.Structure):
    _fields_ = [("extension_base", ExtBase), ("metadata", C.POINTER(Metadata))]


class MockXla:
    """The XLA side of a call: an API table whose callbacks record what a handler asks for."""

    def __init__(self, stream=None, allocate=None):
        self.errors = []        # (code, message) per XLA_FFI_Error_Create
        self.allocations = []   # (size, alignment, pointer)
        self.frees = []         # (size, pointer)
        self.stream_gets = 0
        self._stream = stream
        self._allocate = allocate
        self._cbs = (ERROR_CREATE(self._error_create), STREAM_GET(self._stream_get),
                     ALLOCATE(self._alloc), FREE(self._free))
        self.api = Api()
        self.api.struct_size = C.sizeof(Api)
        self.api.api_version = ApiVersion(C.sizeof(ApiVersion), None, 0, 1)
        self.api.error_create, self.api.stream_get = self._cbs[0], self._cbs[1]
        self.api.device_memory_allocate, self.api.device_memory_free = self._cbs[2], self._cbs[3]

    def _error_create(self, a):
        self.errors.append((a.contents.errc, a.contents.message.decode()))
        return len(self.errors)  # an opaque non-null handle

    def _stream_get(self, a):
        self.stream_gets += 1
        a.contents.stream = self._stream
        return None

    def _alloc(self, a):
        size, align = a.contents.size, a.contents.alignment
        ptr = self._allocate(size, align) if self._allocate else None
        self.allocations.append((size, align, ptr))
        if ptr is None:
            self.errors.append((INTERNAL, "mock: out of memory"))
            return len(self.errors)
        a.contents.data = ptr
        return None

    def _free(self, a):
        self.frees.append((a.contents.size, a.contents.data))
        return None

    def call(self, handler, args, rets, attrs, stage=EXECUTE, extension=None):
        """Call `handler` with buffers given as (dtype, data pointer, dims) and attributes as
        name -> (dtype, value). Returns the handler's XLA_FFI_Error* (None on success)."""
        keep = []

        def buffers(items):
            ptrs = (C.c_void_p * max(len(items), 1))()
            types = (C.c_int * max(len(items), 1))()
            for i, (dtype, data, dims) in enumerate(items):
                d = (C.c_int64 * max(len(dims), 1))(*dims)
                b = Buffer(C.sizeof(Buffer), None, dtype, data, len(dims), d)
                keep.extend((d, b))
                ptrs[i] = C.cast(C.pointer(b), C.c_void_p)
                types[i] = BUFFER
            keep.extend((ptrs, types))
            return Args(C.sizeof(Args), None, len(items), types, ptrs)

        names = (C.POINTER(ByteSpan) * max(len(attrs), 1))()
        values = (C.c_void_p * max(len(attrs), 1))()
        atypes = (C.c_int * max(len(attrs), 1))()
        ctype = {F32: C.c_float, S64: C.c_int64, PRED: C.c_uint8, S32: C.c_int32}
        for i, (name, (dtype, value)) in enumerate(sorted(attrs.items())):
            raw = name.encode()
            span = ByteSpan(raw, len(raw))
            v = ctype[dtype](value)
            sc = Scalar(dtype, C.cast(C.pointer(v), C.c_void_p))
            keep.extend((raw, span, v, sc))
            names[i] = C.pointer(span)
            values[i] = C.cast(C.pointer(sc), C.c_void_p)
            atypes[i] = ATTR_SCALAR
        keep.extend((names, values, atypes))
        frame = CallFrame(C.sizeof(CallFrame), extension, C.pointer(self.api), None, stage,
                          buffers(args), buffers(rets),
                          Attrs(C.sizeof(Attrs), None, len(attrs), atypes, names, values))
        fn = handler
        fn.argtypes = [C.POINTER(CallFrame)]
        fn.restype = C.c_void_p
        return fn(C.byref(frame))


def metadata(handler):
    """(major, minor, traits) that the handler reports to XLA's metadata query."""
    mock = MockXla()
    md = Metadata(C.sizeof(Metadata), ApiVersion(), 0xFFFF)
    ext = MetadataExtension(ExtBase(C.sizeof(MetadataExtension), METADATA, None), C.pointer(md))
    res = mock.call(handler, [], [], {}, extension=C.cast(C.pointer(ext), C.c_void_p))
    assert res is None and not mock.errors
    return md.api_version.major_version, md.api_version.minor_version, md.traits

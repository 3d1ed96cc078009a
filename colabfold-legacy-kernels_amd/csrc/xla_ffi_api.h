// The part of the XLA FFI C ABI (XLA's xla/ffi/api/c_api.h, API version 0.1, the version the
// reference builds against: scripts/build_kernels.sh:53-58 pins jax 0.6.2's headers) that the
// handlers in xla_ffi.cc use. XLA's headers are not available in this build environment, so the
// few structs and enums are declared here with the layout of that public C ABI: every struct
// starts with its size and an extension chain, enums carry XLA's numbering, and the API table
// lists its function pointers in XLA's order. Nothing here is a compatibility layer: these are
// the types the XLA runtime passes to a handler symbol.
#ifndef CLK_XLA_FFI_API_H_
#define CLK_XLA_FFI_API_H_

#include <stddef.h>
#include <stdint.h>

extern "C" {

#define CLK_XLA_FFI_API_MAJOR 0
#define CLK_XLA_FFI_API_MINOR 1

typedef enum { XLA_FFI_Extension_Metadata = 1 } XLA_FFI_Extension_Type;

typedef struct XLA_FFI_Extension_Base {
    size_t struct_size;
    XLA_FFI_Extension_Type type;
    struct XLA_FFI_Extension_Base* next;
} XLA_FFI_Extension_Base;

typedef enum {
    XLA_FFI_ExecutionStage_INSTANTIATE = 0,
    XLA_FFI_ExecutionStage_PREPARE = 1,
    XLA_FFI_ExecutionStage_INITIALIZE = 2,
    XLA_FFI_ExecutionStage_EXECUTE = 3,
} XLA_FFI_ExecutionStage;

// XLA's primitive-type numbering (the subset the targets bind)
typedef enum {
    XLA_FFI_DataType_INVALID = 0,
    XLA_FFI_DataType_PRED = 1,
    XLA_FFI_DataType_S32 = 4,
    XLA_FFI_DataType_S64 = 5,
    XLA_FFI_DataType_U8 = 6,
    XLA_FFI_DataType_F16 = 10,
    XLA_FFI_DataType_F32 = 11,
} XLA_FFI_DataType;

typedef enum {
    XLA_FFI_Error_Code_OK = 0,
    XLA_FFI_Error_Code_INVALID_ARGUMENT = 3,
    XLA_FFI_Error_Code_RESOURCE_EXHAUSTED = 8,
    XLA_FFI_Error_Code_INTERNAL = 13,
} XLA_FFI_Error_Code;

typedef struct XLA_FFI_Error XLA_FFI_Error;                       // opaque, owned by XLA
typedef struct XLA_FFI_ExecutionContext XLA_FFI_ExecutionContext; // opaque
typedef struct XLA_FFI_InternalApi XLA_FFI_InternalApi;           // opaque

typedef struct XLA_FFI_Api_Version {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    int major_version;
    int minor_version;
} XLA_FFI_Api_Version;

typedef struct XLA_FFI_Error_Create_Args {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    const char* message;
    XLA_FFI_Error_Code errc;
} XLA_FFI_Error_Create_Args;

typedef struct XLA_FFI_Stream_Get_Args {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    XLA_FFI_ExecutionContext* ctx;
    void* stream;  // out
} XLA_FFI_Stream_Get_Args;

typedef struct XLA_FFI_DeviceMemory_Allocate_Args {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    XLA_FFI_ExecutionContext* ctx;
    size_t size;
    size_t alignment;
    void* data;  // out
} XLA_FFI_DeviceMemory_Allocate_Args;

typedef struct XLA_FFI_DeviceMemory_Free_Args {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    XLA_FFI_ExecutionContext* ctx;
    size_t size;
    void* data;
} XLA_FFI_DeviceMemory_Free_Args;

typedef XLA_FFI_Error* XLA_FFI_Error_Create(XLA_FFI_Error_Create_Args* args);
typedef XLA_FFI_Error* XLA_FFI_Stream_Get(XLA_FFI_Stream_Get_Args* args);
typedef XLA_FFI_Error* XLA_FFI_DeviceMemory_Allocate(XLA_FFI_DeviceMemory_Allocate_Args* args);
typedef XLA_FFI_Error* XLA_FFI_DeviceMemory_Free(XLA_FFI_DeviceMemory_Free_Args* args);
typedef void XLA_FFI_Unused_Fn(void);  // entries of the table this library does not call

typedef struct XLA_FFI_Api {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    XLA_FFI_Api_Version api_version;
    XLA_FFI_InternalApi* internal_api;
    XLA_FFI_Error_Create* XLA_FFI_Error_Create;
    XLA_FFI_Unused_Fn* XLA_FFI_Error_GetMessage;
    XLA_FFI_Unused_Fn* XLA_FFI_Error_Destroy;
    XLA_FFI_Unused_Fn* XLA_FFI_Handler_Register;
    XLA_FFI_Stream_Get* XLA_FFI_Stream_Get;
    XLA_FFI_Unused_Fn* XLA_FFI_TypeId_Register;
    XLA_FFI_Unused_Fn* XLA_FFI_ExecutionContext_Get;
    XLA_FFI_Unused_Fn* XLA_FFI_State_Set;
    XLA_FFI_Unused_Fn* XLA_FFI_State_Get;
    XLA_FFI_DeviceMemory_Allocate* XLA_FFI_DeviceMemory_Allocate;
    XLA_FFI_DeviceMemory_Free* XLA_FFI_DeviceMemory_Free;
} XLA_FFI_Api;

typedef enum { XLA_FFI_ArgType_BUFFER = 1 } XLA_FFI_ArgType;
typedef enum { XLA_FFI_RetType_BUFFER = 1 } XLA_FFI_RetType;
typedef enum {
    XLA_FFI_AttrType_ARRAY = 1,
    XLA_FFI_AttrType_DICTIONARY = 2,
    XLA_FFI_AttrType_SCALAR = 3,
    XLA_FFI_AttrType_STRING = 4,
} XLA_FFI_AttrType;

typedef struct XLA_FFI_Buffer {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    XLA_FFI_DataType dtype;
    void* data;
    int64_t rank;
    int64_t* dims;
} XLA_FFI_Buffer;

typedef struct XLA_FFI_Args {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    int64_t size;
    XLA_FFI_ArgType* types;
    void** args;
} XLA_FFI_Args;

typedef struct XLA_FFI_Rets {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    int64_t size;
    XLA_FFI_RetType* types;
    void** rets;
} XLA_FFI_Rets;

typedef struct XLA_FFI_ByteSpan {
    const char* ptr;
    size_t len;
} XLA_FFI_ByteSpan;

typedef struct XLA_FFI_Scalar {
    XLA_FFI_DataType dtype;
    void* value;
} XLA_FFI_Scalar;

typedef struct XLA_FFI_Attrs {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    int64_t size;
    XLA_FFI_AttrType* types;
    XLA_FFI_ByteSpan** names;
    void** attrs;
} XLA_FFI_Attrs;

typedef struct XLA_FFI_CallFrame {
    size_t struct_size;
    XLA_FFI_Extension_Base* extension_start;
    const XLA_FFI_Api* api;
    XLA_FFI_ExecutionContext* ctx;
    XLA_FFI_ExecutionStage stage;
    XLA_FFI_Args args;
    XLA_FFI_Rets rets;
    XLA_FFI_Attrs attrs;
} XLA_FFI_CallFrame;

// Handler traits: bit 0 marks a handler that may be recorded into a command buffer (graph).
typedef uint32_t XLA_FFI_Handler_Traits;
#define CLK_XLA_FFI_TRAIT_COMMAND_BUFFER_COMPATIBLE 1u

typedef struct XLA_FFI_Metadata {
    size_t struct_size;
    XLA_FFI_Api_Version api_version;
    XLA_FFI_Handler_Traits traits;
} XLA_FFI_Metadata;

typedef struct XLA_FFI_Metadata_Extension {
    XLA_FFI_Extension_Base extension_base;
    XLA_FFI_Metadata* metadata;
} XLA_FFI_Metadata_Extension;

}  // extern "C"

#endif  // CLK_XLA_FFI_API_H_

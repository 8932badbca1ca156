// pjrt_abi.h -- the part of the PJRT C API (PJRT_API_MAJOR.MINOR = 0.112) this
// plugin implements, restated for this build.
//
// jaxlib binds a plugin through one symbol, GetPjrtApi, returning a table of
// function pointers whose order and whose argument-struct layouts are fixed by
// openxla's xla/pjrt/c/pjrt_c_api.h at that version (the reference vendors it as
// pjrt_plugin/vendor/pjrt_c_api.h; its table is at lines 3016-3186).  Those
// layouts have to match byte for byte, so the structs below keep the field
// order and types of that interface; everything else about this plugin is its
// own.  Every argument struct starts with {struct_size, extension_start}.
#ifndef PJRT_AMD_PJRT_ABI_H_
#define PJRT_AMD_PJRT_ABI_H_

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

extern "C" {

constexpr int kPjrtApiMajor = 0;
constexpr int kPjrtApiMinor = 112;

struct PJRT_Extension_Base {
  size_t struct_size;
  int type;
  PJRT_Extension_Base* next;
};

struct PJRT_Api_Version {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  int major_version;
  int minor_version;
};

// opaque objects: defined by this plugin
struct PJRT_Error;
struct PJRT_Client;
struct PJRT_Device;
struct PJRT_DeviceDescription;
struct PJRT_Memory;
struct PJRT_Executable;
struct PJRT_LoadedExecutable;
struct PJRT_Buffer;
struct PJRT_Event;
struct PJRT_Device_Attributes;
struct PJRT_DeviceAssignmentSerialized;
// PJRT_ExecuteOptions up to the fields this plugin reads (the donation list)
struct PJRT_ExecuteOptions {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  void** send_callbacks;
  void** recv_callbacks;
  size_t num_send_ops;
  size_t num_recv_ops;
  int launch_id;
  const int64_t* non_donatable_input_indices;
  size_t num_non_donatable_input_indices;
};
struct PJRT_Buffer_MemoryLayout;

enum PJRT_Error_Code {
  PJRT_Error_Code_OK = 0,
  PJRT_Error_Code_CANCELLED = 1,
  PJRT_Error_Code_UNKNOWN = 2,
  PJRT_Error_Code_INVALID_ARGUMENT = 3,
  PJRT_Error_Code_DEADLINE_EXCEEDED = 4,
  PJRT_Error_Code_NOT_FOUND = 5,
  PJRT_Error_Code_ALREADY_EXISTS = 6,
  PJRT_Error_Code_PERMISSION_DENIED = 7,
  PJRT_Error_Code_RESOURCE_EXHAUSTED = 8,
  PJRT_Error_Code_FAILED_PRECONDITION = 9,
  PJRT_Error_Code_ABORTED = 10,
  PJRT_Error_Code_OUT_OF_RANGE = 11,
  PJRT_Error_Code_UNIMPLEMENTED = 12,
  PJRT_Error_Code_INTERNAL = 13,
  PJRT_Error_Code_UNAVAILABLE = 14,
  PJRT_Error_Code_DATA_LOSS = 15,
  PJRT_Error_Code_UNAUTHENTICATED = 16,
};

enum PJRT_NamedValue_Type {
  PJRT_NamedValue_kString = 0,
  PJRT_NamedValue_kInt64 = 1,
  PJRT_NamedValue_kInt64List = 2,
  PJRT_NamedValue_kFloat = 3,
  PJRT_NamedValue_kBool = 4,
};

// element types (the values this plugin produces or accepts)
enum PJRT_Buffer_Type {
  PJRT_Buffer_Type_INVALID = 0,
  PJRT_Buffer_Type_PRED = 1,
  PJRT_Buffer_Type_S8 = 2,
  PJRT_Buffer_Type_S16 = 3,
  PJRT_Buffer_Type_S32 = 4,
  PJRT_Buffer_Type_S64 = 5,
  PJRT_Buffer_Type_U8 = 6,
  PJRT_Buffer_Type_U16 = 7,
  PJRT_Buffer_Type_U32 = 8,
  PJRT_Buffer_Type_U64 = 9,
  PJRT_Buffer_Type_F16 = 10,
  PJRT_Buffer_Type_F32 = 11,
  PJRT_Buffer_Type_F64 = 12,
  PJRT_Buffer_Type_BF16 = 13,
};

enum PJRT_HostBufferSemantics {
  PJRT_HostBufferSemantics_kImmutableOnlyDuringCall = 0,
  PJRT_HostBufferSemantics_kImmutableUntilTransferCompletes = 1,
  PJRT_HostBufferSemantics_kImmutableZeroCopy = 2,
  PJRT_HostBufferSemantics_kMutableZeroCopy = 3,
};

struct PJRT_NamedValue {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const char* name;
  size_t name_size;
  PJRT_NamedValue_Type type;
  union {
    const char* string_value;
    int64_t int64_value;
    const int64_t* int64_array_value;
    float float_value;
    bool bool_value;
  };
  size_t value_size;
};

struct PJRT_Program {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  char* code;
  size_t code_size;
  const char* format;
  size_t format_size;
};

struct PJRT_LogicalDeviceIds {
  int replica;
  int partition;
};

typedef void (*PJRT_Error_PayloadVisitor)(const char* key, size_t key_size, const char* value, size_t value_size,
                                          void* user_arg);
typedef void (*PJRT_Event_OnReadyCallback)(PJRT_Error* error, void* user_arg);

#define PJRT_ARGS_HEAD          \
  size_t struct_size;           \
  PJRT_Extension_Base* extension_start

// ---- errors ----
struct PJRT_Error_Destroy_Args { PJRT_ARGS_HEAD; PJRT_Error* error; };
struct PJRT_Error_Message_Args { PJRT_ARGS_HEAD; const PJRT_Error* error; const char* message; size_t message_size; };
struct PJRT_Error_GetCode_Args { PJRT_ARGS_HEAD; const PJRT_Error* error; PJRT_Error_Code code; };
struct PJRT_Error_ForEachPayload_Args {
  PJRT_ARGS_HEAD;
  const PJRT_Error* error;
  PJRT_Error_PayloadVisitor visitor;
  void* user_arg;
};

// ---- plugin ----
struct PJRT_Plugin_Initialize_Args { PJRT_ARGS_HEAD; };
struct PJRT_Plugin_Attributes_Args { PJRT_ARGS_HEAD; const PJRT_NamedValue* attributes; size_t num_attributes; };

// ---- events ----
struct PJRT_Event_Destroy_Args { PJRT_ARGS_HEAD; PJRT_Event* event; };
struct PJRT_Event_IsReady_Args { PJRT_ARGS_HEAD; PJRT_Event* event; bool is_ready; };
struct PJRT_Event_Error_Args { PJRT_ARGS_HEAD; PJRT_Event* event; };
struct PJRT_Event_Await_Args { PJRT_ARGS_HEAD; PJRT_Event* event; };
struct PJRT_Event_OnReady_Args { PJRT_ARGS_HEAD; PJRT_Event* event; PJRT_Event_OnReadyCallback callback; void* user_arg; };

// ---- client ----
struct PJRT_Client_Create_Args {
  PJRT_ARGS_HEAD;
  const PJRT_NamedValue* create_options;
  size_t num_options;
  void* kv_get_callback;
  void* kv_get_user_arg;
  void* kv_put_callback;
  void* kv_put_user_arg;
  PJRT_Client* client;
  void* kv_try_get_callback;
  void* kv_try_get_user_arg;
};
struct PJRT_Client_Destroy_Args { PJRT_ARGS_HEAD; PJRT_Client* client; };
struct PJRT_Client_PlatformName_Args { PJRT_ARGS_HEAD; PJRT_Client* client; const char* platform_name; size_t platform_name_size; };
struct PJRT_Client_ProcessIndex_Args { PJRT_ARGS_HEAD; PJRT_Client* client; int process_index; };
struct PJRT_Client_PlatformVersion_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const char* platform_version;
  size_t platform_version_size;
};
struct PJRT_Client_Devices_Args { PJRT_ARGS_HEAD; PJRT_Client* client; PJRT_Device* const* devices; size_t num_devices; };
struct PJRT_Client_AddressableDevices_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  PJRT_Device* const* addressable_devices;
  size_t num_addressable_devices;
};
struct PJRT_Client_LookupDevice_Args { PJRT_ARGS_HEAD; PJRT_Client* client; int id; PJRT_Device* device; };
struct PJRT_Client_LookupAddressableDevice_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  int local_hardware_id;
  PJRT_Device* addressable_device;
};
struct PJRT_Client_AddressableMemories_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  PJRT_Memory* const* addressable_memories;
  size_t num_addressable_memories;
};
struct PJRT_Client_Compile_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const PJRT_Program* program;
  const char* compile_options;
  size_t compile_options_size;
  PJRT_LoadedExecutable* executable;
};
struct PJRT_Client_DefaultDeviceAssignment_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  int num_replicas;
  int num_partitions;
  size_t default_assignment_size;
  int* default_assignment;
};
struct PJRT_Client_BufferFromHostBuffer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const void* data;
  PJRT_Buffer_Type type;
  const int64_t* dims;
  size_t num_dims;
  const int64_t* byte_strides;
  size_t num_byte_strides;
  PJRT_HostBufferSemantics host_buffer_semantics;
  PJRT_Device* device;
  PJRT_Memory* memory;
  PJRT_Buffer_MemoryLayout* device_layout;
  PJRT_Event* done_with_host_buffer;
  PJRT_Buffer* buffer;
};

// ---- device description / device / memory ----
struct PJRT_DeviceDescription_Id_Args { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; int id; };
struct PJRT_DeviceDescription_ProcessIndex_Args { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; int process_index; };
struct PJRT_DeviceDescription_Attributes_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  size_t num_attributes;
  const PJRT_NamedValue* attributes;
};
struct PJRT_DeviceDescription_String_Args {   // Kind, DebugString, ToString share this layout
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  const char* text;
  size_t text_size;
};
struct PJRT_Device_GetDescription_Args { PJRT_ARGS_HEAD; PJRT_Device* device; PJRT_DeviceDescription* device_description; };
struct PJRT_Device_IsAddressable_Args { PJRT_ARGS_HEAD; PJRT_Device* device; bool is_addressable; };
struct PJRT_Device_LocalHardwareId_Args { PJRT_ARGS_HEAD; PJRT_Device* device; int local_hardware_id; };
struct PJRT_Device_AddressableMemories_Args { PJRT_ARGS_HEAD; PJRT_Device* device; PJRT_Memory* const* memories; size_t num_memories; };
struct PJRT_Device_DefaultMemory_Args { PJRT_ARGS_HEAD; PJRT_Device* device; PJRT_Memory* memory; };
struct PJRT_Device_GetAttributes_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  const PJRT_NamedValue* attributes;
  size_t num_attributes;
  PJRT_Device_Attributes* device_attributes;
  void (*attributes_deleter)(PJRT_Device_Attributes* device_attributes);
};
struct PJRT_Memory_Id_Args { PJRT_ARGS_HEAD; PJRT_Memory* memory; int id; };
struct PJRT_Memory_String_Args { PJRT_ARGS_HEAD; PJRT_Memory* memory; const char* text; size_t text_size; };   // Kind, DebugString, ToString
struct PJRT_Memory_AddressableByDevices_Args { PJRT_ARGS_HEAD; PJRT_Memory* memory; PJRT_Device* const* devices; size_t num_devices; };
struct PJRT_Memory_Kind_Id_Args { PJRT_ARGS_HEAD; PJRT_Memory* memory; int kind_id; };

// ---- executables ----
struct PJRT_Executable_Destroy_Args { PJRT_ARGS_HEAD; PJRT_Executable* executable; };
struct PJRT_Executable_Name_Args { PJRT_ARGS_HEAD; PJRT_Executable* executable; const char* executable_name; size_t executable_name_size; };
struct PJRT_Executable_Count_Args { PJRT_ARGS_HEAD; PJRT_Executable* executable; size_t count; };   // NumReplicas / NumPartitions / NumOutputs
struct PJRT_Executable_SizeOfGeneratedCodeInBytes_Args { PJRT_ARGS_HEAD; PJRT_Executable* executable; int64_t size_in_bytes; };
struct PJRT_Executable_OutputElementTypes_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  PJRT_Buffer_Type* output_types;
  size_t num_output_types;
};
struct PJRT_Executable_OutputDimensions_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_outputs;
  const int64_t* dims;
  const size_t* dim_sizes;
};
struct PJRT_Executable_OutputMemoryKinds_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_outputs;
  const char* const* memory_kinds;
  const size_t* memory_kind_sizes;
};
struct PJRT_Executable_Fingerprint_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  const char* executable_fingerprint;
  size_t executable_fingerprint_size;
};
struct PJRT_LoadedExecutable_Destroy_Args { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; };
struct PJRT_LoadedExecutable_GetExecutable_Args { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* loaded_executable; PJRT_Executable* executable; };
struct PJRT_LoadedExecutable_AddressableDevices_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  PJRT_Device* const* addressable_devices;
  size_t num_addressable_devices;
};
struct PJRT_LoadedExecutable_Delete_Args { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; };
struct PJRT_LoadedExecutable_IsDeleted_Args { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; bool is_deleted; };
struct PJRT_LoadedExecutable_Execute_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  PJRT_ExecuteOptions* options;
  PJRT_Buffer* const* const* argument_lists;
  size_t num_devices;
  size_t num_args;
  PJRT_Buffer** const* output_lists;
  PJRT_Event** device_complete_events;
  PJRT_Device* execute_device;
};
struct PJRT_LoadedExecutable_AddressableDeviceLogicalIds_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  PJRT_LogicalDeviceIds* addressable_device_logical_ids;
  size_t num_addressable_device_logical_ids;
};
struct PJRT_LoadedExecutable_GetDeviceAssignment_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  const char* serialized_bytes;
  size_t serialized_bytes_size;
  PJRT_DeviceAssignmentSerialized* serialized_device_assignment;
  void (*serialized_device_assignment_deleter)(PJRT_DeviceAssignmentSerialized* da);
};
struct PJRT_LoadedExecutable_Fingerprint_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  const char* executable_fingerprint;
  size_t executable_fingerprint_size;
};

// ---- buffers ----
struct PJRT_Buffer_Destroy_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; };
struct PJRT_Buffer_ElementType_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Buffer_Type type; };
struct PJRT_Buffer_Dimensions_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; const int64_t* dims; size_t num_dims; };
struct PJRT_Buffer_DynamicDimensionIndices_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  const size_t* dynamic_dim_indices;
  size_t num_dynamic_dims;
};
struct PJRT_Buffer_OnDeviceSizeInBytes_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; size_t on_device_size_in_bytes; };
struct PJRT_Buffer_Device_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Device* device; };
struct PJRT_Buffer_Memory_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Memory* memory; };
struct PJRT_Buffer_Delete_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; };
struct PJRT_Buffer_IsDeleted_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; bool is_deleted; };
struct PJRT_Buffer_ToHostBuffer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* src;
  PJRT_Buffer_MemoryLayout* host_layout;
  void* dst;
  size_t dst_size;
  PJRT_Event* event;
};
struct PJRT_Buffer_IsOnCpu_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; bool is_on_cpu; };
struct PJRT_Buffer_ReadyEvent_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Event* event; };
struct PJRT_Buffer_UnsafePointer_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; uintptr_t buffer_pointer; };
struct PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; void* device_memory_ptr; };

#undef PJRT_ARGS_HEAD

// ---- the function table: slot names in the interface's order --------------------------
#define PJRT_AMD_API_SLOTS(X)                                                                                  \
  X(PJRT_Error_Destroy) X(PJRT_Error_Message) X(PJRT_Error_GetCode) X(PJRT_Plugin_Initialize)                  \
  X(PJRT_Plugin_Attributes) X(PJRT_Event_Destroy) X(PJRT_Event_IsReady) X(PJRT_Event_Error) X(PJRT_Event_Await)  \
  X(PJRT_Event_OnReady) X(PJRT_Client_Create) X(PJRT_Client_Destroy) X(PJRT_Client_PlatformName)                \
  X(PJRT_Client_ProcessIndex) X(PJRT_Client_PlatformVersion) X(PJRT_Client_Devices)                             \
  X(PJRT_Client_AddressableDevices) X(PJRT_Client_LookupDevice) X(PJRT_Client_LookupAddressableDevice)          \
  X(PJRT_Client_AddressableMemories) X(PJRT_Client_Compile) X(PJRT_Client_DefaultDeviceAssignment)              \
  X(PJRT_Client_BufferFromHostBuffer) X(PJRT_DeviceDescription_Id) X(PJRT_DeviceDescription_ProcessIndex)       \
  X(PJRT_DeviceDescription_Attributes) X(PJRT_DeviceDescription_Kind) X(PJRT_DeviceDescription_DebugString)     \
  X(PJRT_DeviceDescription_ToString) X(PJRT_Device_GetDescription) X(PJRT_Device_IsAddressable)                 \
  X(PJRT_Device_LocalHardwareId) X(PJRT_Device_AddressableMemories) X(PJRT_Device_DefaultMemory)                \
  X(PJRT_Device_MemoryStats) X(PJRT_Memory_Id) X(PJRT_Memory_Kind) X(PJRT_Memory_DebugString)                   \
  X(PJRT_Memory_ToString) X(PJRT_Memory_AddressableByDevices) X(PJRT_Executable_Destroy)                        \
  X(PJRT_Executable_Name) X(PJRT_Executable_NumReplicas) X(PJRT_Executable_NumPartitions)                       \
  X(PJRT_Executable_NumOutputs) X(PJRT_Executable_SizeOfGeneratedCodeInBytes) X(PJRT_Executable_GetCostAnalysis) \
  X(PJRT_Executable_OutputMemoryKinds) X(PJRT_Executable_OptimizedProgram) X(PJRT_Executable_Serialize)         \
  X(PJRT_LoadedExecutable_Destroy) X(PJRT_LoadedExecutable_GetExecutable)                                       \
  X(PJRT_LoadedExecutable_AddressableDevices) X(PJRT_LoadedExecutable_Delete) X(PJRT_LoadedExecutable_IsDeleted) \
  X(PJRT_LoadedExecutable_Execute) X(PJRT_Executable_DeserializeAndLoad) X(PJRT_LoadedExecutable_Fingerprint)   \
  X(PJRT_Buffer_Destroy) X(PJRT_Buffer_ElementType) X(PJRT_Buffer_Dimensions) X(PJRT_Buffer_UnpaddedDimensions)  \
  X(PJRT_Buffer_DynamicDimensionIndices) X(PJRT_Buffer_GetMemoryLayout) X(PJRT_Buffer_OnDeviceSizeInBytes)      \
  X(PJRT_Buffer_Device) X(PJRT_Buffer_Memory) X(PJRT_Buffer_Delete) X(PJRT_Buffer_IsDeleted)                     \
  X(PJRT_Buffer_CopyToDevice) X(PJRT_Buffer_ToHostBuffer) X(PJRT_Buffer_IsOnCpu) X(PJRT_Buffer_ReadyEvent)       \
  X(PJRT_Buffer_UnsafePointer) X(PJRT_Buffer_IncreaseExternalReferenceCount)                                    \
  X(PJRT_Buffer_DecreaseExternalReferenceCount) X(PJRT_Buffer_OpaqueDeviceMemoryDataPointer)                    \
  X(PJRT_CopyToDeviceStream_Destroy) X(PJRT_CopyToDeviceStream_AddChunk) X(PJRT_CopyToDeviceStream_TotalBytes)   \
  X(PJRT_CopyToDeviceStream_GranuleSize) X(PJRT_CopyToDeviceStream_CurrentBytes)                                \
  X(PJRT_TopologyDescription_Create) X(PJRT_TopologyDescription_Destroy)                                        \
  X(PJRT_TopologyDescription_PlatformName) X(PJRT_TopologyDescription_PlatformVersion)                          \
  X(PJRT_TopologyDescription_GetDeviceDescriptions) X(PJRT_TopologyDescription_Serialize)                       \
  X(PJRT_TopologyDescription_Attributes) X(PJRT_Compile) X(PJRT_Executable_OutputElementTypes)                  \
  X(PJRT_Executable_OutputDimensions) X(PJRT_Buffer_CopyToMemory) X(PJRT_Client_CreateViewOfDeviceBuffer)        \
  X(PJRT_Executable_Fingerprint) X(PJRT_Client_TopologyDescription) X(PJRT_Executable_GetCompiledMemoryStats)   \
  X(PJRT_Memory_Kind_Id) X(PJRT_ExecuteContext_Create) X(PJRT_ExecuteContext_Destroy)                           \
  X(PJRT_Buffer_CopyRawToHost) X(PJRT_AsyncHostToDeviceTransferManager_Destroy)                                 \
  X(PJRT_AsyncHostToDeviceTransferManager_TransferData) X(PJRT_Client_CreateBuffersForAsyncHostToDevice)        \
  X(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer) X(PJRT_AsyncHostToDeviceTransferManager_Device)       \
  X(PJRT_AsyncHostToDeviceTransferManager_BufferCount) X(PJRT_AsyncHostToDeviceTransferManager_BufferSize)      \
  X(PJRT_AsyncHostToDeviceTransferManager_SetBufferError) X(PJRT_AsyncHostToDeviceTransferManager_AddMetadata)  \
  X(PJRT_Client_DmaMap) X(PJRT_Client_DmaUnmap) X(PJRT_Client_CreateUninitializedBuffer)                        \
  X(PJRT_Client_UpdateGlobalProcessInfo) X(PJRT_TopologyDescription_Deserialize) X(PJRT_Client_CreateAliasBuffer) \
  X(PJRT_Client_FulfillAliasBuffer) X(PJRT_LoadedExecutable_GetDeviceAssignment) X(PJRT_Client_CreateErrorBuffer) \
  X(PJRT_AsyncHostToDeviceTransferManager_TransferLiteral) X(PJRT_Buffer_CopyRawToHostFuture)                   \
  X(PJRT_Device_PoisonExecution) X(PJRT_Device_CreateAsyncTrackingEvent) X(PJRT_AsyncTrackingEvent_Destroy)     \
  X(PJRT_Executable_GetCompileOptions) X(PJRT_Buffer_DonateWithControlDependency) X(PJRT_Event_Create)          \
  X(PJRT_Event_Set) X(PJRT_Device_GetAttributes) X(PJRT_Client_Load)                                           \
  X(PJRT_LoadedExecutable_AddressableDeviceLogicalIds) X(PJRT_Buffer_Bitcast) X(PJRT_Error_ForEachPayload)      \
  X(PJRT_TopologyDescription_Fingerprint) X(PJRT_Executable_ParameterMemoryKinds) X(PJRT_Device_ClearMemoryStats) \
  X(PJRT_TopologyDescription_MakeCanonicalShapeForMemorySpace) X(PJRT_TopologyDescription_GetMemorySpaceKindIds)

enum PjrtAmdSlot {
#define PJRT_AMD_SLOT_ENUM(name) kSlot_##name,
  PJRT_AMD_API_SLOTS(PJRT_AMD_SLOT_ENUM)
#undef PJRT_AMD_SLOT_ENUM
      kSlotCount
};

// Every slot but the first two (Error_Destroy, Error_Message: void) returns
// PJRT_Error* and takes one argument struct; the table stores them untyped.
typedef void (*PjrtSlot)(void);

struct PJRT_Api {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Api_Version pjrt_api_version;
  PjrtSlot slots[kSlotCount];
};

const PJRT_Api* GetPjrtApi(void);

}  // extern "C"

#endif  // PJRT_AMD_PJRT_ABI_H_

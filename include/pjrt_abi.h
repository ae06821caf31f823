/*
 * pjrt_abi.h — the PJRT C API (OpenXLA, version 0.90) as this plugin binds it.
 *
 * jaxlib and other PJRT clients call a plugin only through the function table
 * returned by GetPjrtApi() and through the argument structs of each entry, so
 * the table's slot order and every argument struct's field order below must
 * match PJRT C API 0.90 exactly (the reference plugin compiles against that
 * version: reference third_party/xla/pjrt/c/pjrt_c_api.h:92,107, table at
 * :2758-2915).  Argument structs are declared for the entries this plugin
 * implements; the remaining table slots are typed generically (every slot is
 * one function pointer, so the layout is unaffected).
 *
 * Conventions of the API: every entry returns NULL on success or a
 * plugin-allocated PJRT_Error the caller frees with PJRT_Error_Destroy; each
 * argument struct starts with struct_size (the caller's sizeof) and an
 * extension chain pointer.
 */
#ifndef PJRT_ABI_H_
#define PJRT_ABI_H_

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PJRT_ABI_MAJOR 0
#define PJRT_ABI_MINOR 90

/* Size a struct had when `last` was its final field (used for struct_size). */
#define PJRT_ABI_SIZE(type, last) (offsetof(type, last) + sizeof(((type*)0)->last))

typedef struct PJRT_Error PJRT_Error;
typedef struct PJRT_Event PJRT_Event;
typedef struct PJRT_Client PJRT_Client;
typedef struct PJRT_Device PJRT_Device;
typedef struct PJRT_Memory PJRT_Memory;
typedef struct PJRT_DeviceDescription PJRT_DeviceDescription;
typedef struct PJRT_TopologyDescription PJRT_TopologyDescription;
typedef struct PJRT_Executable PJRT_Executable;
typedef struct PJRT_LoadedExecutable PJRT_LoadedExecutable;
typedef struct PJRT_Buffer PJRT_Buffer;
typedef struct PJRT_ExecuteContext PJRT_ExecuteContext;
typedef struct PJRT_SerializedExecutable PJRT_SerializedExecutable;
typedef struct PJRT_DeviceAssignmentSerialized PJRT_DeviceAssignmentSerialized;
typedef struct PJRT_SerializedTopology PJRT_SerializedTopology;

typedef struct PJRT_Extension_Base {
  size_t struct_size;
  int type; /* PJRT_Extension_Type */
  struct PJRT_Extension_Base* next;
} PJRT_Extension_Base;

typedef struct PJRT_Api_Version {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  int major_version;
  int minor_version;
} PJRT_Api_Version;

typedef enum {
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
  PJRT_Error_Code_UNAUTHENTICATED = 16
} PJRT_Error_Code;

/* Element types: the order is the ABI. */
typedef enum {
  PJRT_Buffer_Type_INVALID,
  PJRT_Buffer_Type_PRED,
  PJRT_Buffer_Type_S8,
  PJRT_Buffer_Type_S16,
  PJRT_Buffer_Type_S32,
  PJRT_Buffer_Type_S64,
  PJRT_Buffer_Type_U8,
  PJRT_Buffer_Type_U16,
  PJRT_Buffer_Type_U32,
  PJRT_Buffer_Type_U64,
  PJRT_Buffer_Type_F16,
  PJRT_Buffer_Type_F32,
  PJRT_Buffer_Type_F64,
  PJRT_Buffer_Type_BF16,
  PJRT_Buffer_Type_C64,
  PJRT_Buffer_Type_C128,
  PJRT_Buffer_Type_F8E5M2,
  PJRT_Buffer_Type_F8E4M3FN,
  PJRT_Buffer_Type_F8E4M3B11FNUZ,
  PJRT_Buffer_Type_F8E5M2FNUZ,
  PJRT_Buffer_Type_F8E4M3FNUZ,
  PJRT_Buffer_Type_S4,
  PJRT_Buffer_Type_U4,
  PJRT_Buffer_Type_TOKEN,
  PJRT_Buffer_Type_S2,
  PJRT_Buffer_Type_U2,
  PJRT_Buffer_Type_F8E4M3,
  PJRT_Buffer_Type_F8E3M4,
  PJRT_Buffer_Type_F8E8M0FNU,
  PJRT_Buffer_Type_F4E2M1FN
} PJRT_Buffer_Type;

typedef enum {
  PJRT_HostBufferSemantics_kImmutableOnlyDuringCall,
  PJRT_HostBufferSemantics_kImmutableUntilTransferCompletes,
  PJRT_HostBufferSemantics_kImmutableZeroCopy,
  PJRT_HostBufferSemantics_kMutableZeroCopy
} PJRT_HostBufferSemantics;

typedef enum {
  PJRT_NamedValue_kString = 0,
  PJRT_NamedValue_kInt64,
  PJRT_NamedValue_kInt64List,
  PJRT_NamedValue_kFloat,
  PJRT_NamedValue_kBool
} PJRT_NamedValue_Type;

typedef struct PJRT_NamedValue {
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
} PJRT_NamedValue;

typedef enum {
  PJRT_Buffer_MemoryLayout_Type_Tiled = 0,
  PJRT_Buffer_MemoryLayout_Type_Strides
} PJRT_Buffer_MemoryLayout_Type;

typedef struct PJRT_Buffer_MemoryLayout_Tiled {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const int64_t* minor_to_major;
  size_t minor_to_major_size;
  const int64_t* tile_dims;
  const size_t* tile_dim_sizes;
  size_t num_tiles;
} PJRT_Buffer_MemoryLayout_Tiled;

typedef struct PJRT_Buffer_MemoryLayout_Strides {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  const int64_t* byte_strides;
  size_t num_byte_strides;
} PJRT_Buffer_MemoryLayout_Strides;

typedef struct PJRT_Buffer_MemoryLayout {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  union {
    PJRT_Buffer_MemoryLayout_Tiled tiled;
    PJRT_Buffer_MemoryLayout_Strides strides;
  };
  PJRT_Buffer_MemoryLayout_Type type;
} PJRT_Buffer_MemoryLayout;

/* ---- argument structs (field order = ABI) ------------------------------- */

#define PJRT_ARGS_HEAD          \
  size_t struct_size;           \
  PJRT_Extension_Base* extension_start

typedef struct { PJRT_ARGS_HEAD; PJRT_Error* error; } PJRT_Error_Destroy_Args;
typedef struct { PJRT_ARGS_HEAD; const PJRT_Error* error; const char* message; size_t message_size; } PJRT_Error_Message_Args;
typedef struct { PJRT_ARGS_HEAD; const PJRT_Error* error; PJRT_Error_Code code; } PJRT_Error_GetCode_Args;

typedef struct { PJRT_ARGS_HEAD; } PJRT_Plugin_Initialize_Args;
typedef struct { PJRT_ARGS_HEAD; const PJRT_NamedValue* attributes; size_t num_attributes; } PJRT_Plugin_Attributes_Args;

typedef void (*PJRT_Event_OnReadyCallback)(PJRT_Error* error, void* user_arg);
typedef struct { PJRT_ARGS_HEAD; PJRT_Event* event; } PJRT_Event_Destroy_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Event* event; bool is_ready; } PJRT_Event_IsReady_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Event* event; } PJRT_Event_Error_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Event* event; } PJRT_Event_Await_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Event* event; PJRT_Event_OnReadyCallback callback; void* user_arg; } PJRT_Event_OnReady_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Event* event; } PJRT_Event_Create_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Event* event; PJRT_Error_Code error_code; const char* error_message; size_t error_message_size; } PJRT_Event_Set_Args;

typedef struct {
  PJRT_ARGS_HEAD;
  const PJRT_NamedValue* create_options;
  size_t num_options;
  void* kv_get_callback;
  void* kv_get_user_arg;
  void* kv_put_callback;
  void* kv_put_user_arg;
  PJRT_Client* client; /* out */
  void* kv_try_get_callback;
  void* kv_try_get_user_arg;
} PJRT_Client_Create_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; } PJRT_Client_Destroy_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; const char* platform_name; size_t platform_name_size; } PJRT_Client_PlatformName_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; int process_index; } PJRT_Client_ProcessIndex_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; const char* platform_version; size_t platform_version_size; } PJRT_Client_PlatformVersion_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; PJRT_TopologyDescription* topology; } PJRT_Client_TopologyDescription_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; PJRT_Device* const* devices; size_t num_devices; } PJRT_Client_Devices_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; PJRT_Device* const* addressable_devices; size_t num_addressable_devices; } PJRT_Client_AddressableDevices_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; int id; PJRT_Device* device; } PJRT_Client_LookupDevice_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; int local_hardware_id; PJRT_Device* addressable_device; } PJRT_Client_LookupAddressableDevice_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Client* client; PJRT_Memory* const* addressable_memories; size_t num_addressable_memories; } PJRT_Client_AddressableMemories_Args;

typedef struct {
  PJRT_ARGS_HEAD;
  char* code;
  size_t code_size;
  const char* format;
  size_t format_size;
} PJRT_Program;

typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const PJRT_Program* program;
  const char* compile_options;
  size_t compile_options_size;
  PJRT_LoadedExecutable* executable; /* out */
} PJRT_Client_Compile_Args;

typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  int num_replicas;
  int num_partitions;
  size_t default_assignment_size;
  int* default_assignment;
} PJRT_Client_DefaultDeviceAssignment_Args;

typedef struct {
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
  PJRT_Event* done_with_host_buffer; /* out */
  PJRT_Buffer* buffer;               /* out */
} PJRT_Client_BufferFromHostBuffer_Args;

typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  void* device_buffer_ptr;
  const int64_t* dims;
  size_t num_dims;
  PJRT_Buffer_Type element_type;
  PJRT_Buffer_MemoryLayout* layout;
  PJRT_Device* device;
  void (*on_delete_callback)(void* device_buffer_ptr, void* user_arg);
  void* on_delete_callback_arg;
  intptr_t stream;
  PJRT_Buffer* buffer; /* out */
  PJRT_Memory* memory;
} PJRT_Client_CreateViewOfDeviceBuffer_Args;

typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const int64_t* shape_dims;
  size_t shape_num_dims;
  PJRT_Buffer_Type shape_element_type;
  PJRT_Buffer_MemoryLayout* shape_layout;
  PJRT_Device* device;
  PJRT_Memory* memory;
  PJRT_Buffer* buffer; /* out */
} PJRT_Client_CreateUninitializedBuffer_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; int id; } PJRT_DeviceDescription_Id_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; int process_index; } PJRT_DeviceDescription_ProcessIndex_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; size_t num_attributes; const PJRT_NamedValue* attributes; } PJRT_DeviceDescription_Attributes_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; const char* device_kind; size_t device_kind_size; } PJRT_DeviceDescription_Kind_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; const char* debug_string; size_t debug_string_size; } PJRT_DeviceDescription_DebugString_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_DeviceDescription* device_description; const char* to_string; size_t to_string_size; } PJRT_DeviceDescription_ToString_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_Device* device; PJRT_DeviceDescription* device_description; } PJRT_Device_GetDescription_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Device* device; bool is_addressable; } PJRT_Device_IsAddressable_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Device* device; int local_hardware_id; } PJRT_Device_LocalHardwareId_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Device* device; PJRT_Memory* const* memories; size_t num_memories; } PJRT_Device_AddressableMemories_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Device* device; PJRT_Memory* memory; } PJRT_Device_DefaultMemory_Args;
typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  int64_t bytes_in_use;
  int64_t peak_bytes_in_use;
  bool peak_bytes_in_use_is_set;
  int64_t num_allocs;
  bool num_allocs_is_set;
  int64_t largest_alloc_size;
  bool largest_alloc_size_is_set;
  int64_t bytes_limit;
  bool bytes_limit_is_set;
  int64_t bytes_reserved;
  bool bytes_reserved_is_set;
  int64_t peak_bytes_reserved;
  bool peak_bytes_reserved_is_set;
  int64_t bytes_reservable_limit;
  bool bytes_reservable_limit_is_set;
  int64_t largest_free_block_bytes;
  bool largest_free_block_bytes_is_set;
  int64_t pool_bytes;
  bool pool_bytes_is_set;
  int64_t peak_pool_bytes;
  bool peak_pool_bytes_is_set;
} PJRT_Device_MemoryStats_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_Memory* memory; int id; } PJRT_Memory_Id_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Memory* memory; const char* kind; size_t kind_size; } PJRT_Memory_Kind_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Memory* memory; int kind_id; } PJRT_Memory_Kind_Id_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Memory* memory; const char* debug_string; size_t debug_string_size; } PJRT_Memory_DebugString_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Memory* memory; const char* to_string; size_t to_string_size; } PJRT_Memory_ToString_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Memory* memory; PJRT_Device* const* devices; size_t num_devices; } PJRT_Memory_AddressableByDevices_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_ExecuteContext* context; } PJRT_ExecuteContext_Create_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_ExecuteContext* context; } PJRT_ExecuteContext_Destroy_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; } PJRT_Executable_Destroy_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; } PJRT_LoadedExecutable_Destroy_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* loaded_executable; PJRT_Executable* executable; } PJRT_LoadedExecutable_GetExecutable_Args;
typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  const char* serialized_bytes;
  size_t serialized_bytes_size;
  PJRT_DeviceAssignmentSerialized* serialized_device_assignment;
  void (*serialized_device_assignment_deleter)(PJRT_DeviceAssignmentSerialized* da);
} PJRT_LoadedExecutable_GetDeviceAssignment_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; const char* executable_name; size_t executable_name_size; } PJRT_Executable_Name_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; size_t num_replicas; } PJRT_Executable_NumReplicas_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; size_t num_partitions; } PJRT_Executable_NumPartitions_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; PJRT_Device* const* addressable_devices; size_t num_addressable_devices; } PJRT_LoadedExecutable_AddressableDevices_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; PJRT_Program* program; } PJRT_Executable_OptimizedProgram_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; } PJRT_LoadedExecutable_Delete_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; bool is_deleted; } PJRT_LoadedExecutable_IsDeleted_Args;

typedef struct {
  PJRT_ARGS_HEAD;
  void** send_callbacks;
  void** recv_callbacks;
  size_t num_send_ops;
  size_t num_recv_ops;
  int launch_id;
  const int64_t* non_donatable_input_indices;
  size_t num_non_donatable_input_indices;
  PJRT_ExecuteContext* context;
  const char* call_location;
  size_t num_tasks;
  int* task_ids;
  int64_t* incarnation_ids;
} PJRT_ExecuteOptions;

typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  PJRT_ExecuteOptions* options;
  PJRT_Buffer* const* const* argument_lists; /* [num_devices][num_args] */
  size_t num_devices;
  size_t num_args;
  PJRT_Buffer** const* output_lists;         /* [num_devices][num_outputs], plugin fills */
  PJRT_Event** device_complete_events;       /* optional [num_devices], plugin fills */
  PJRT_Device* execute_device;
} PJRT_LoadedExecutable_Execute_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; size_t num_outputs; } PJRT_Executable_NumOutputs_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; int64_t size_in_bytes; } PJRT_Executable_SizeOfGeneratedCodeInBytes_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; const char* executable_fingerprint; size_t executable_fingerprint_size; } PJRT_Executable_Fingerprint_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; size_t num_properties; const PJRT_NamedValue* properties; } PJRT_Executable_GetCostAnalysis_Args;
typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  int64_t generated_code_size_in_bytes;
  int64_t argument_size_in_bytes;
  int64_t output_size_in_bytes;
  int64_t alias_size_in_bytes;
  int64_t temp_size_in_bytes;
  int64_t host_generated_code_size_in_bytes;
  int64_t host_argument_size_in_bytes;
  int64_t host_output_size_in_bytes;
  int64_t host_alias_size_in_bytes;
  int64_t host_temp_size_in_bytes;
  int64_t peak_memory_in_bytes;
  int64_t total_size_in_bytes;
} PJRT_Executable_GetCompiledMemoryStats_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; PJRT_Buffer_Type* output_types; size_t num_output_types; } PJRT_Executable_OutputElementTypes_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; size_t num_outputs; const int64_t* dims; const size_t* dim_sizes; } PJRT_Executable_OutputDimensions_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Executable* executable; size_t num_outputs; const char* const* memory_kinds; const size_t* memory_kind_sizes; } PJRT_Executable_OutputMemoryKinds_Args;
typedef struct {
  PJRT_ARGS_HEAD;
  const PJRT_Executable* executable;
  const char* serialized_bytes;
  size_t serialized_bytes_size;
  PJRT_SerializedExecutable* serialized_executable;
  void (*serialized_executable_deleter)(PJRT_SerializedExecutable* exec);
} PJRT_Executable_Serialize_Args;
typedef struct {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const char* serialized_executable;
  size_t serialized_executable_size;
  PJRT_LoadedExecutable* loaded_executable; /* out */
  const char* overridden_serialized_compile_options;
  size_t overridden_serialized_compile_options_size;
} PJRT_Executable_DeserializeAndLoad_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_LoadedExecutable* executable; const char* executable_fingerprint; size_t executable_fingerprint_size; } PJRT_LoadedExecutable_Fingerprint_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; } PJRT_Buffer_Destroy_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Buffer_Type type; } PJRT_Buffer_ElementType_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; const int64_t* dims; size_t num_dims; } PJRT_Buffer_Dimensions_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; const int64_t* unpadded_dims; size_t num_dims; } PJRT_Buffer_UnpaddedDimensions_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; const size_t* dynamic_dim_indices; size_t num_dynamic_dims; } PJRT_Buffer_DynamicDimensionIndices_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Buffer_MemoryLayout layout; } PJRT_Buffer_GetMemoryLayout_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* src; PJRT_Buffer_MemoryLayout* host_layout; void* dst; size_t dst_size; PJRT_Event* event; } PJRT_Buffer_ToHostBuffer_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; size_t on_device_size_in_bytes; } PJRT_Buffer_OnDeviceSizeInBytes_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; } PJRT_Buffer_Delete_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; bool is_deleted; } PJRT_Buffer_IsDeleted_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; void* dst; int64_t offset; int64_t transfer_size; PJRT_Event* event; } PJRT_Buffer_CopyRawToHost_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Device* dst_device; PJRT_Buffer* dst_buffer; } PJRT_Buffer_CopyToDevice_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Memory* dst_memory; PJRT_Buffer* dst_buffer; } PJRT_Buffer_CopyToMemory_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; bool is_on_cpu; } PJRT_Buffer_IsOnCpu_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Device* device; } PJRT_Buffer_Device_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Memory* memory; } PJRT_Buffer_Memory_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; PJRT_Event* event; } PJRT_Buffer_ReadyEvent_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; uintptr_t buffer_pointer; } PJRT_Buffer_UnsafePointer_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; } PJRT_Buffer_IncreaseExternalReferenceCount_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; } PJRT_Buffer_DecreaseExternalReferenceCount_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_Buffer* buffer; void* device_memory_ptr; } PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args;

typedef struct { PJRT_ARGS_HEAD; PJRT_TopologyDescription* topology; } PJRT_TopologyDescription_Destroy_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_TopologyDescription* topology; const char* platform_version; size_t platform_version_size; } PJRT_TopologyDescription_PlatformVersion_Args;
typedef struct { PJRT_ARGS_HEAD; const PJRT_TopologyDescription* topology; const char* platform_name; size_t platform_name_size; } PJRT_TopologyDescription_PlatformName_Args;
typedef struct { PJRT_ARGS_HEAD; const PJRT_TopologyDescription* topology; PJRT_DeviceDescription* const* descriptions; size_t num_descriptions; } PJRT_TopologyDescription_GetDeviceDescriptions_Args;
typedef struct { PJRT_ARGS_HEAD; PJRT_TopologyDescription* topology; const PJRT_NamedValue* attributes; size_t num_attributes; } PJRT_TopologyDescription_Attributes_Args;

/* ---- the function table --------------------------------------------------- */

/* Slots this plugin answers only with an UNIMPLEMENTED error. */
typedef PJRT_Error* (*PJRT_UnimplementedFn)(void* args);

#define PJRT_FN(name) PJRT_Error* (*name)(name##_Args * args)
#define PJRT_STUB(name) PJRT_UnimplementedFn name

typedef struct PJRT_Api {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Api_Version pjrt_api_version;

  void (*PJRT_Error_Destroy)(PJRT_Error_Destroy_Args* args);
  void (*PJRT_Error_Message)(PJRT_Error_Message_Args* args);
  PJRT_FN(PJRT_Error_GetCode);

  PJRT_FN(PJRT_Plugin_Initialize);
  PJRT_FN(PJRT_Plugin_Attributes);

  PJRT_FN(PJRT_Event_Destroy);
  PJRT_FN(PJRT_Event_IsReady);
  PJRT_FN(PJRT_Event_Error);
  PJRT_FN(PJRT_Event_Await);
  PJRT_FN(PJRT_Event_OnReady);

  PJRT_FN(PJRT_Client_Create);
  PJRT_FN(PJRT_Client_Destroy);
  PJRT_FN(PJRT_Client_PlatformName);
  PJRT_FN(PJRT_Client_ProcessIndex);
  PJRT_FN(PJRT_Client_PlatformVersion);
  PJRT_FN(PJRT_Client_Devices);
  PJRT_FN(PJRT_Client_AddressableDevices);
  PJRT_FN(PJRT_Client_LookupDevice);
  PJRT_FN(PJRT_Client_LookupAddressableDevice);
  PJRT_FN(PJRT_Client_AddressableMemories);
  PJRT_FN(PJRT_Client_Compile);
  PJRT_FN(PJRT_Client_DefaultDeviceAssignment);
  PJRT_FN(PJRT_Client_BufferFromHostBuffer);

  PJRT_FN(PJRT_DeviceDescription_Id);
  PJRT_FN(PJRT_DeviceDescription_ProcessIndex);
  PJRT_FN(PJRT_DeviceDescription_Attributes);
  PJRT_FN(PJRT_DeviceDescription_Kind);
  PJRT_FN(PJRT_DeviceDescription_DebugString);
  PJRT_FN(PJRT_DeviceDescription_ToString);

  PJRT_FN(PJRT_Device_GetDescription);
  PJRT_FN(PJRT_Device_IsAddressable);
  PJRT_FN(PJRT_Device_LocalHardwareId);
  PJRT_FN(PJRT_Device_AddressableMemories);
  PJRT_FN(PJRT_Device_DefaultMemory);
  PJRT_FN(PJRT_Device_MemoryStats);

  PJRT_FN(PJRT_Memory_Id);
  PJRT_FN(PJRT_Memory_Kind);
  PJRT_FN(PJRT_Memory_DebugString);
  PJRT_FN(PJRT_Memory_ToString);
  PJRT_FN(PJRT_Memory_AddressableByDevices);

  PJRT_FN(PJRT_Executable_Destroy);
  PJRT_FN(PJRT_Executable_Name);
  PJRT_FN(PJRT_Executable_NumReplicas);
  PJRT_FN(PJRT_Executable_NumPartitions);
  PJRT_FN(PJRT_Executable_NumOutputs);
  PJRT_FN(PJRT_Executable_SizeOfGeneratedCodeInBytes);
  PJRT_FN(PJRT_Executable_GetCostAnalysis);
  PJRT_FN(PJRT_Executable_OutputMemoryKinds);
  PJRT_FN(PJRT_Executable_OptimizedProgram);
  PJRT_FN(PJRT_Executable_Serialize);

  PJRT_FN(PJRT_LoadedExecutable_Destroy);
  PJRT_FN(PJRT_LoadedExecutable_GetExecutable);
  PJRT_FN(PJRT_LoadedExecutable_AddressableDevices);
  PJRT_FN(PJRT_LoadedExecutable_Delete);
  PJRT_FN(PJRT_LoadedExecutable_IsDeleted);
  PJRT_FN(PJRT_LoadedExecutable_Execute);
  PJRT_FN(PJRT_Executable_DeserializeAndLoad);
  PJRT_FN(PJRT_LoadedExecutable_Fingerprint);

  PJRT_FN(PJRT_Buffer_Destroy);
  PJRT_FN(PJRT_Buffer_ElementType);
  PJRT_FN(PJRT_Buffer_Dimensions);
  PJRT_FN(PJRT_Buffer_UnpaddedDimensions);
  PJRT_FN(PJRT_Buffer_DynamicDimensionIndices);
  PJRT_FN(PJRT_Buffer_GetMemoryLayout);
  PJRT_FN(PJRT_Buffer_OnDeviceSizeInBytes);
  PJRT_FN(PJRT_Buffer_Device);
  PJRT_FN(PJRT_Buffer_Memory);
  PJRT_FN(PJRT_Buffer_Delete);
  PJRT_FN(PJRT_Buffer_IsDeleted);
  PJRT_FN(PJRT_Buffer_CopyToDevice);
  PJRT_FN(PJRT_Buffer_ToHostBuffer);
  PJRT_FN(PJRT_Buffer_IsOnCpu);
  PJRT_FN(PJRT_Buffer_ReadyEvent);
  PJRT_FN(PJRT_Buffer_UnsafePointer);
  PJRT_FN(PJRT_Buffer_IncreaseExternalReferenceCount);
  PJRT_FN(PJRT_Buffer_DecreaseExternalReferenceCount);
  PJRT_FN(PJRT_Buffer_OpaqueDeviceMemoryDataPointer);

  PJRT_STUB(PJRT_CopyToDeviceStream_Destroy);
  PJRT_STUB(PJRT_CopyToDeviceStream_AddChunk);
  PJRT_STUB(PJRT_CopyToDeviceStream_TotalBytes);
  PJRT_STUB(PJRT_CopyToDeviceStream_GranuleSize);
  PJRT_STUB(PJRT_CopyToDeviceStream_CurrentBytes);

  PJRT_STUB(PJRT_TopologyDescription_Create);
  PJRT_FN(PJRT_TopologyDescription_Destroy);
  PJRT_FN(PJRT_TopologyDescription_PlatformName);
  PJRT_FN(PJRT_TopologyDescription_PlatformVersion);
  PJRT_FN(PJRT_TopologyDescription_GetDeviceDescriptions);
  PJRT_STUB(PJRT_TopologyDescription_Serialize);
  PJRT_FN(PJRT_TopologyDescription_Attributes);

  PJRT_STUB(PJRT_Compile);

  PJRT_FN(PJRT_Executable_OutputElementTypes);
  PJRT_FN(PJRT_Executable_OutputDimensions);

  PJRT_FN(PJRT_Buffer_CopyToMemory);

  PJRT_FN(PJRT_Client_CreateViewOfDeviceBuffer);

  PJRT_FN(PJRT_Executable_Fingerprint);

  PJRT_FN(PJRT_Client_TopologyDescription);

  PJRT_FN(PJRT_Executable_GetCompiledMemoryStats);

  PJRT_FN(PJRT_Memory_Kind_Id);

  PJRT_FN(PJRT_ExecuteContext_Create);
  PJRT_FN(PJRT_ExecuteContext_Destroy);
  PJRT_FN(PJRT_Buffer_CopyRawToHost);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_Destroy);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_TransferData);
  PJRT_STUB(PJRT_Client_CreateBuffersForAsyncHostToDevice);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_Device);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_BufferCount);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_BufferSize);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_SetBufferError);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_AddMetadata);
  PJRT_STUB(PJRT_Client_DmaMap);
  PJRT_STUB(PJRT_Client_DmaUnmap);

  PJRT_FN(PJRT_Client_CreateUninitializedBuffer);
  PJRT_STUB(PJRT_Client_UpdateGlobalProcessInfo);
  PJRT_STUB(PJRT_TopologyDescription_Deserialize);
  PJRT_STUB(PJRT_Client_CreateAliasBuffer);
  PJRT_STUB(PJRT_Client_FulfillAliasBuffer);
  PJRT_FN(PJRT_LoadedExecutable_GetDeviceAssignment);
  PJRT_STUB(PJRT_Client_CreateErrorBuffer);
  PJRT_STUB(PJRT_AsyncHostToDeviceTransferManager_TransferLiteral);
  PJRT_STUB(PJRT_Buffer_CopyRawToHostFuture);
  PJRT_STUB(PJRT_Device_PoisonExecution);
  PJRT_STUB(PJRT_Device_CreateAsyncTrackingEvent);
  PJRT_STUB(PJRT_AsyncTrackingEvent_Destroy);
  PJRT_STUB(PJRT_Executable_GetCompileOptions);
  PJRT_STUB(PJRT_Buffer_DonateWithControlDependency);
  PJRT_FN(PJRT_Event_Create);
  PJRT_FN(PJRT_Event_Set);
} PJRT_Api;

#undef PJRT_FN
#undef PJRT_STUB

/* Number of function slots in the 0.90 table (checked by the plugin). */
#define PJRT_ABI_NUM_SLOTS 128

#ifdef __cplusplus
}
#endif

#endif /* PJRT_ABI_H_ */

// PJRT C API 0.90 implementation: the plugin's object model and GetPjrtApi.
//
// Replaces the reference's PJRT surface (reference src/jax_mlx_pjrt.cpp:
// 533-1650, 8920-9670) for one HIP device per PJRT device:
//   * buffers are hipMalloc'd device memory (memory kind "device", not on the
//     CPU), recycled through a per-client size-bucketed pool;
//   * Compile parses MLIR text (or MLIR bytecode via the in-process jaxlib),
//     inlines calls, rewrites the fused patterns and builds a static launch
//     plan; Execute replays it on the client's HIP stream and returns outputs
//     whose ready events are real hipEvents;
//   * output element types and dimensions are the module's true ones
//     (the reference reports F32 and leaves dimensions unset,
//     src/jax_mlx_pjrt.cpp:1466-1526);
//   * host buffers honour byte_strides, argument structs are size-checked,
//     client state is guarded by a mutex, and no per-call files are written.
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "ir.h"
#include "pjrt_mi355x.h"
#include "plan.h"

#define MFXP_EXPORT __attribute__((visibility("default")))

namespace mfxp {
// bytecode.cpp
bool program_text(const char* data, size_t size, std::string& text, std::string& route, std::string& err);
}  // namespace mfxp

using namespace mfxp;

// ---------------------------------------------------------------------------
// Errors

struct PJRT_Error {
  PJRT_Error_Code code;
  std::string message;
};

namespace {

PJRT_Error* make_error(PJRT_Error_Code code, const std::string& msg) {
  return new PJRT_Error{code, msg};
}
PJRT_Error* unimplemented(const char* what) {
  return make_error(PJRT_Error_Code_UNIMPLEMENTED, std::string(what) + " is not implemented by the MI355X plugin");
}
PJRT_Error* hip_error(hipError_t e, const char* what) {
  return make_error(PJRT_Error_Code_INTERNAL, std::string(what) + ": " + hipGetErrorString(e));
}

#define CHECK_ARGS(type, last)                                                                   \
  do {                                                                                           \
    if (!args) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, #type ": null args");         \
    if (args->struct_size < PJRT_ABI_SIZE(type, last))                                           \
      return make_error(PJRT_Error_Code_INVALID_ARGUMENT,                                        \
                        std::string(#type ": struct_size ") + std::to_string(args->struct_size) + \
                            " is smaller than expected " +                                        \
                            std::to_string(PJRT_ABI_SIZE(type, last)));                           \
  } while (0)

#define GUARD_BEGIN try {
#define GUARD_END                                                         \
  }                                                                       \
  catch (const std::exception& e) {                                       \
    return make_error(PJRT_Error_Code_INTERNAL, e.what());                \
  }                                                                       \
  catch (...) {                                                           \
    return make_error(PJRT_Error_Code_INTERNAL, "unknown C++ exception"); \
  }

// ---------------------------------------------------------------------------
// dtype mapping

DType from_pjrt(PJRT_Buffer_Type t) {
  switch (t) {
    case PJRT_Buffer_Type_PRED: return DType::kPred;
    case PJRT_Buffer_Type_S8: return DType::kI8;
    case PJRT_Buffer_Type_S16: return DType::kI16;
    case PJRT_Buffer_Type_S32: return DType::kI32;
    case PJRT_Buffer_Type_S64: return DType::kI64;
    case PJRT_Buffer_Type_U8: return DType::kU8;
    case PJRT_Buffer_Type_U16: return DType::kU16;
    case PJRT_Buffer_Type_U32: return DType::kU32;
    case PJRT_Buffer_Type_U64: return DType::kU64;
    case PJRT_Buffer_Type_F16: return DType::kF16;
    case PJRT_Buffer_Type_F32: return DType::kF32;
    case PJRT_Buffer_Type_F64: return DType::kF64;
    case PJRT_Buffer_Type_BF16: return DType::kBF16;
    default: return DType::kInvalid;
  }
}

PJRT_Buffer_Type to_pjrt(DType t) {
  switch (t) {
    case DType::kPred: return PJRT_Buffer_Type_PRED;
    case DType::kI8: return PJRT_Buffer_Type_S8;
    case DType::kI16: return PJRT_Buffer_Type_S16;
    case DType::kI32: return PJRT_Buffer_Type_S32;
    case DType::kI64: return PJRT_Buffer_Type_S64;
    case DType::kU8: return PJRT_Buffer_Type_U8;
    case DType::kU16: return PJRT_Buffer_Type_U16;
    case DType::kU32: return PJRT_Buffer_Type_U32;
    case DType::kU64: return PJRT_Buffer_Type_U64;
    case DType::kF16: return PJRT_Buffer_Type_F16;
    case DType::kF32: return PJRT_Buffer_Type_F32;
    case DType::kF64: return PJRT_Buffer_Type_F64;
    case DType::kBF16: return PJRT_Buffer_Type_BF16;
    default: return PJRT_Buffer_Type_INVALID;
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Object model

struct EventState {
  hipEvent_t ev = nullptr;  // null: ready at creation
  std::mutex mu;
  bool set = true;          // user events: false until PJRT_Event_Set
  PJRT_Error_Code code = PJRT_Error_Code_OK;
  std::string message;
  ~EventState() {
    if (ev) (void)hipEventDestroy(ev);
  }
};

struct PJRT_Event {
  std::shared_ptr<EventState> st;
};

struct PJRT_DeviceDescription {
  int id = 0;
  int ordinal = 0;
  std::string kind, debug, tostr, arch;
  int64_t core_count = 0;
  std::vector<PJRT_NamedValue> attrs;
};

struct PJRT_Memory {
  int id = 0;
  std::string kind = "device", debug, tostr;
  std::vector<PJRT_Device*> devices;
};

struct PJRT_Client;

struct PJRT_Device {
  PJRT_DeviceDescription desc;
  PJRT_Memory* memory = nullptr;
  PJRT_Client* client = nullptr;
  int ordinal = 0;
  hipStream_t stream = nullptr;
};

struct PJRT_TopologyDescription {
  PJRT_Client* client = nullptr;
  std::vector<PJRT_DeviceDescription*> descs;
};

// The client is reference counted: Client_Destroy drops the owner's reference
// and every buffer and loaded executable holds one, so buffers a caller frees
// after the client (jaxlib's teardown order is not guaranteed, nor is
// Python's garbage collection) still return their memory to a live pool.
struct PJRT_Client {
  std::atomic<int> refs{1};
  void ref() { ++refs; }
  void unref() {
    if (--refs == 0) delete this;
  }
  std::vector<std::unique_ptr<PJRT_Device>> devices;
  std::vector<std::unique_ptr<PJRT_Memory>> memories;
  std::vector<PJRT_Device*> device_ptrs;
  std::vector<PJRT_Memory*> memory_ptrs;
  PJRT_TopologyDescription topology;
  std::string platform_name = "mi355x";
  std::string platform_version;
  std::mutex mu;
  // Size-bucketed pool of device allocations (stream-ordered reuse: every
  // kernel of this client runs on its device's single stream).
  std::map<std::pair<int, size_t>, std::vector<void*>> pool;

  void* alloc(int ordinal, size_t bytes, hipError_t& e) {
    size_t b = bytes < 256 ? 256 : (bytes + 255) / 256 * 256;
    {
      std::lock_guard<std::mutex> lock(mu);
      auto it = pool.find({ordinal, b});
      if (it != pool.end() && !it->second.empty()) {
        void* p = it->second.back();
        it->second.pop_back();
        e = hipSuccess;
        return p;
      }
    }
    void* p = nullptr;
    e = hipSetDevice(ordinal);
    if (e == hipSuccess) e = hipMalloc(&p, b);
    return e == hipSuccess ? p : nullptr;
  }
  void release(int ordinal, void* p, size_t bytes) {
    size_t b = bytes < 256 ? 256 : (bytes + 255) / 256 * 256;
    std::lock_guard<std::mutex> lock(mu);
    pool[{ordinal, b}].push_back(p);
  }
  ~PJRT_Client() {
    for (auto& d : devices) {
      (void)hipSetDevice(d->ordinal);
      (void)hipStreamSynchronize(d->stream);
    }
    for (auto& kv : pool)
      for (void* p : kv.second) (void)hipFree(p);
    for (auto& d : devices)
      if (d->stream) (void)hipStreamDestroy(d->stream);
  }
};

// One counted reference to a client.
class ClientRef {
 public:
  ClientRef() = default;
  ClientRef(const ClientRef&) = delete;
  ClientRef& operator=(const ClientRef&) = delete;
  ~ClientRef() { reset(); }
  ClientRef& operator=(PJRT_Client* c) {
    if (c) c->ref();
    reset();
    p_ = c;
    return *this;
  }
  void reset() {
    if (p_) p_->unref();
    p_ = nullptr;
  }
  PJRT_Client* operator->() const { return p_; }
  operator PJRT_Client*() const { return p_; }

 private:
  PJRT_Client* p_ = nullptr;
};

struct PJRT_Buffer {
  ClientRef client;
  PJRT_Device* device = nullptr;
  void* ptr = nullptr;
  size_t bytes = 0;
  mfxp::Type type;
  bool owned = true;
  bool deleted = false;
  std::atomic<int> ext_refs{0};
  std::shared_ptr<EventState> ready;
  void (*on_delete)(void*, void*) = nullptr;
  void* on_delete_arg = nullptr;
  std::vector<int64_t> minor_to_major;

  // Set when the memory's release waits for the last external reference,
  // and when Buffer_Destroy came while one was still held (the object then
  // lives until that reference is dropped).
  bool release_pending = false;
  bool destroyed = false;
  std::mutex mu;

  // Marks the buffer deleted and releases its memory: owned memory returns to
  // the client's stream-ordered pool (later work on the stream reuses it only
  // after the work already queued), a view's on_delete callback runs once the
  // work queued on the device's stream has finished reading it.  While
  // external references (DLPack and the like) are held, the release waits for
  // the last one to be dropped.
  void free_memory() {
    std::lock_guard<std::mutex> g(mu);
    if (deleted) return;
    deleted = true;
    if (ext_refs.load() > 0) {
      release_pending = true;
      return;
    }
    release_locked();
  }
  void release_locked() {
    if (owned && ptr) {
      client->release(device->ordinal, ptr, bytes);
    } else if (on_delete) {
      if (device && device->stream) (void)hipStreamSynchronize(device->stream);
      on_delete(ptr, on_delete_arg);
    }
    ptr = nullptr;
    release_pending = false;
  }
};

struct PJRT_Executable {
  std::atomic<int> refs{1};
  std::string name, fingerprint;
  std::string text;  // the MLIR text the plan was built from (Serialize)
  std::unique_ptr<Plan> plan;
  std::vector<PJRT_Buffer_Type> out_types;
  std::vector<int64_t> out_dims;
  std::vector<size_t> out_dim_sizes;
  std::vector<const char*> mem_kinds;
  std::vector<size_t> mem_kind_sizes;
  std::vector<PJRT_NamedValue> cost;
  std::string json;
  void unref() {
    if (--refs == 0) delete this;
  }
};

struct PJRT_LoadedExecutable {
  PJRT_Executable* exe = nullptr;
  ClientRef client;
  bool deleted = false;
};

struct PJRT_ExecuteContext {};

namespace {

const char* kMemoryKind = "device";

PJRT_Error* event_error(const EventState& st) {
  if (st.code == PJRT_Error_Code_OK) return nullptr;
  return make_error(st.code, st.message);
}

std::shared_ptr<EventState> record_event(hipStream_t s, PJRT_Error** err) {
  auto st = std::make_shared<EventState>();
  hipError_t e = hipEventCreateWithFlags(&st->ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(st->ev, s);
  if (e != hipSuccess) {
    *err = hip_error(e, "hipEventRecord");
    st->ev = nullptr;
  }
  return st;
}

PJRT_Error* wait_event(EventState& st) {
  {
    std::unique_lock<std::mutex> lock(st.mu);
    if (!st.set) return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "awaiting an event that was never set");
  }
  if (st.ev) {
    hipError_t e = hipEventSynchronize(st.ev);
    if (e != hipSuccess) return hip_error(e, "hipEventSynchronize");
  }
  return event_error(st);
}

std::string fnv1a_hex(const std::string& s) {
  uint64_t h = 1469598103934665603ULL;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ULL;
  }
  char buf[17];
  std::snprintf(buf, sizeof buf, "%016llx", (unsigned long long)h);
  return buf;
}

// ---- compile pipeline shared by Client_Compile and mfx_pjrt_inspect --------

struct Compiled {
  std::shared_ptr<Function> main;
  RewriteStats stats;
  std::unique_ptr<Plan> plan;
  std::string module_name;
};

Compiled compile_text(const std::string& text) {
  Module m = parse_module(text);
  verify_module(m);
  inline_calls(m);
  Compiled c;
  c.module_name = m.name;
  c.main = m.main();
  if (!c.main) throw ParseError("module has no main function");
  c.stats = rewrite(*c.main);
  compact(*c.main);
  c.plan = Plan::build(*c.main);
  return c;
}

// ---------------------------------------------------------------------------
// Error / plugin / event

void Error_Destroy(PJRT_Error_Destroy_Args* args) {
  if (args && args->error) delete args->error;
}

void Error_Message(PJRT_Error_Message_Args* args) {
  if (!args || !args->error) return;
  args->message = args->error->message.c_str();
  args->message_size = args->error->message.size();
}

PJRT_Error* Error_GetCode(PJRT_Error_GetCode_Args* args) {
  CHECK_ARGS(PJRT_Error_GetCode_Args, code);
  args->code = args->error ? args->error->code : PJRT_Error_Code_OK;
  return nullptr;
}

PJRT_Error* Plugin_Initialize(PJRT_Plugin_Initialize_Args* args) { return nullptr; }

PJRT_Error* Plugin_Attributes(PJRT_Plugin_Attributes_Args* args) {
  CHECK_ARGS(PJRT_Plugin_Attributes_Args, num_attributes);
  static const int64_t cur[3] = {1, 9, 0};
  static const int64_t min[3] = {0, 9, 0};
  static PJRT_NamedValue attrs[3];
  static std::once_flag once;
  std::call_once(once, [] {
    auto set_list = [](PJRT_NamedValue& nv, const char* name, const int64_t* v, size_t n) {
      std::memset(&nv, 0, sizeof nv);
      nv.struct_size = sizeof(PJRT_NamedValue);
      nv.name = name;
      nv.name_size = std::strlen(name);
      nv.type = PJRT_NamedValue_kInt64List;
      nv.int64_array_value = v;
      nv.value_size = n;
    };
    set_list(attrs[0], "stablehlo_current_version", cur, 3);
    set_list(attrs[1], "stablehlo_minimum_version", min, 3);
    std::memset(&attrs[2], 0, sizeof attrs[2]);
    attrs[2].struct_size = sizeof(PJRT_NamedValue);
    attrs[2].name = "xla_version";
    attrs[2].name_size = std::strlen("xla_version");
    attrs[2].type = PJRT_NamedValue_kInt64;
    attrs[2].int64_value = 2;
    attrs[2].value_size = 1;
  });
  args->attributes = attrs;
  args->num_attributes = 3;
  return nullptr;
}

PJRT_Error* Event_Destroy(PJRT_Event_Destroy_Args* args) {
  CHECK_ARGS(PJRT_Event_Destroy_Args, event);
  delete args->event;
  return nullptr;
}

PJRT_Error* Event_IsReady(PJRT_Event_IsReady_Args* args) {
  CHECK_ARGS(PJRT_Event_IsReady_Args, is_ready);
  EventState& st = *args->event->st;
  {
    std::lock_guard<std::mutex> lock(st.mu);
    if (!st.set) {
      args->is_ready = false;
      return nullptr;
    }
  }
  if (!st.ev) {
    args->is_ready = true;
    return nullptr;
  }
  hipError_t e = hipEventQuery(st.ev);
  if (e == hipErrorNotReady) {
    args->is_ready = false;
    return nullptr;
  }
  if (e != hipSuccess) return hip_error(e, "hipEventQuery");
  args->is_ready = true;
  return nullptr;
}

PJRT_Error* Event_Error(PJRT_Event_Error_Args* args) {
  CHECK_ARGS(PJRT_Event_Error_Args, event);
  return event_error(*args->event->st);
}

PJRT_Error* Event_Await(PJRT_Event_Await_Args* args) {
  CHECK_ARGS(PJRT_Event_Await_Args, event);
  return wait_event(*args->event->st);
}

PJRT_Error* Event_OnReady(PJRT_Event_OnReady_Args* args) {
  CHECK_ARGS(PJRT_Event_OnReady_Args, user_arg);
  // Completion is observed synchronously; the callback owns the error it gets.
  PJRT_Error* err = wait_event(*args->event->st);
  args->callback(err, args->user_arg);
  return nullptr;
}

PJRT_Error* Event_Create(PJRT_Event_Create_Args* args) {
  CHECK_ARGS(PJRT_Event_Create_Args, event);
  auto st = std::make_shared<EventState>();
  st->set = false;
  args->event = new PJRT_Event{st};
  return nullptr;
}

PJRT_Error* Event_Set(PJRT_Event_Set_Args* args) {
  CHECK_ARGS(PJRT_Event_Set_Args, error_message_size);
  EventState& st = *args->event->st;
  std::lock_guard<std::mutex> lock(st.mu);
  st.set = true;
  st.code = args->error_code;
  if (args->error_message) st.message.assign(args->error_message, args->error_message_size);
  return nullptr;
}

// ---------------------------------------------------------------------------
// Client

PJRT_Error* Client_Create(PJRT_Client_Create_Args* args) {
  CHECK_ARGS(PJRT_Client_Create_Args, client);
  GUARD_BEGIN
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "no HIP device is visible (the MI355X plugin needs a GPU)");
  }
  auto c = std::make_unique<PJRT_Client>();
  int rt = 0;
  (void)hipRuntimeGetVersion(&rt);
  c->platform_version = "ROCm HIP runtime " + std::to_string(rt) + ", gfx950 kernels";
  for (int i = 0; i < n; ++i) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, i);
    if (e != hipSuccess) return hip_error(e, "hipGetDeviceProperties");
    auto d = std::make_unique<PJRT_Device>();
    d->ordinal = i;
    d->client = c.get();
    d->desc.id = i;
    d->desc.ordinal = i;
    d->desc.arch = prop.gcnArchName;
    d->desc.kind = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    d->desc.debug = "MI355X:" + std::to_string(i);
    d->desc.tostr = "MI355XDevice(id=" + std::to_string(i) + ", arch=" + d->desc.arch + ")";
    d->desc.core_count = prop.multiProcessorCount;
    // Non-blocking: launches on this stream do not order themselves after
    // the legacy null stream (that implicit wait put a gap of several us
    // before every launch).  Work the plugin depends on is ordered
    // explicitly: host copies run on this stream, and a device view waits
    // for its producer's stream (CreateViewOfDeviceBuffer).  Default priority.
    e = hipSetDevice(i);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_error(e, "hipStreamCreateWithFlags");
    auto m = std::make_unique<PJRT_Memory>();
    m->id = i;
    m->debug = "device memory of MI355X:" + std::to_string(i);
    m->tostr = "MemorySpace(device, id=" + std::to_string(i) + ")";
    m->devices.push_back(d.get());
    d->memory = m.get();
    c->device_ptrs.push_back(d.get());
    c->memory_ptrs.push_back(m.get());
    c->topology.descs.push_back(&d->desc);
    c->devices.push_back(std::move(d));
    c->memories.push_back(std::move(m));
  }
  for (auto& d : c->devices) {
    auto& a = d->desc.attrs;
    a.resize(2);
    std::memset(a.data(), 0, sizeof(PJRT_NamedValue) * a.size());
    a[0].struct_size = sizeof(PJRT_NamedValue);
    a[0].name = "device_vendor";
    a[0].name_size = std::strlen("device_vendor");
    a[0].type = PJRT_NamedValue_kString;
    a[0].string_value = "AMD";
    a[0].value_size = 3;
    a[1].struct_size = sizeof(PJRT_NamedValue);
    a[1].name = "core_count";
    a[1].name_size = std::strlen("core_count");
    a[1].type = PJRT_NamedValue_kInt64;
    a[1].int64_value = d->desc.core_count;
    a[1].value_size = 1;
  }
  (void)hipSetDevice(0);
  c->topology.client = c.get();
  args->client = c.release();
  return nullptr;
  GUARD_END
}

PJRT_Error* Client_Destroy(PJRT_Client_Destroy_Args* args) {
  CHECK_ARGS(PJRT_Client_Destroy_Args, client);
  if (args->client) args->client->unref();
  return nullptr;
}

PJRT_Error* Client_PlatformName(PJRT_Client_PlatformName_Args* args) {
  CHECK_ARGS(PJRT_Client_PlatformName_Args, platform_name_size);
  args->platform_name = args->client->platform_name.c_str();
  args->platform_name_size = args->client->platform_name.size();
  return nullptr;
}

PJRT_Error* Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* args) {
  CHECK_ARGS(PJRT_Client_ProcessIndex_Args, process_index);
  args->process_index = 0;
  return nullptr;
}

PJRT_Error* Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* args) {
  CHECK_ARGS(PJRT_Client_PlatformVersion_Args, platform_version_size);
  args->platform_version = args->client->platform_version.c_str();
  args->platform_version_size = args->client->platform_version.size();
  return nullptr;
}

PJRT_Error* Client_TopologyDescription(PJRT_Client_TopologyDescription_Args* args) {
  CHECK_ARGS(PJRT_Client_TopologyDescription_Args, topology);
  args->topology = &args->client->topology;
  return nullptr;
}

PJRT_Error* Client_Devices(PJRT_Client_Devices_Args* args) {
  CHECK_ARGS(PJRT_Client_Devices_Args, num_devices);
  args->devices = args->client->device_ptrs.data();
  args->num_devices = args->client->device_ptrs.size();
  return nullptr;
}

PJRT_Error* Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* args) {
  CHECK_ARGS(PJRT_Client_AddressableDevices_Args, num_addressable_devices);
  args->addressable_devices = args->client->device_ptrs.data();
  args->num_addressable_devices = args->client->device_ptrs.size();
  return nullptr;
}

PJRT_Error* Client_LookupDevice(PJRT_Client_LookupDevice_Args* args) {
  CHECK_ARGS(PJRT_Client_LookupDevice_Args, device);
  auto& d = args->client->device_ptrs;
  if (args->id < 0 || args->id >= (int)d.size())
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "no device with id " + std::to_string(args->id));
  args->device = d[args->id];
  return nullptr;
}

PJRT_Error* Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* args) {
  CHECK_ARGS(PJRT_Client_LookupAddressableDevice_Args, addressable_device);
  auto& d = args->client->device_ptrs;
  if (args->local_hardware_id < 0 || args->local_hardware_id >= (int)d.size())
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT,
                      "no addressable device " + std::to_string(args->local_hardware_id));
  args->addressable_device = d[args->local_hardware_id];
  return nullptr;
}

PJRT_Error* Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* args) {
  CHECK_ARGS(PJRT_Client_AddressableMemories_Args, num_addressable_memories);
  args->addressable_memories = args->client->memory_ptrs.data();
  args->num_addressable_memories = args->client->memory_ptrs.size();
  return nullptr;
}

PJRT_Error* load_text(PJRT_Client* client, const std::string& text, PJRT_LoadedExecutable** out);

PJRT_Error* Client_Compile(PJRT_Client_Compile_Args* args) {
  CHECK_ARGS(PJRT_Client_Compile_Args, executable);
  GUARD_BEGIN
  const PJRT_Program* prog = args->program;
  if (!prog || !prog->code) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Compile: no program");
  std::string format(prog->format ? prog->format : "", prog->format ? prog->format_size : 0);
  if (format != "mlir")
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Compile: program format '" + format + "' (expected 'mlir')");
  std::string text, route, err;
  if (!program_text(prog->code, prog->code_size, text, route, err))
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "Compile: MLIR bytecode: " + err);
  return load_text(args->client, text, &args->executable);
  GUARD_END
}

// Plans `text` for `client` (Client_Compile and DeserializeAndLoad).
PJRT_Error* load_text(PJRT_Client* client, const std::string& text, PJRT_LoadedExecutable** out) {
  Compiled c;
  try {
    c = compile_text(text);
  } catch (const ParseError& e) {
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, e.what());
  }
  auto* exe = new PJRT_Executable();
  exe->name = c.module_name.empty() ? "main" : c.module_name;
  exe->text = text;
  exe->fingerprint = fnv1a_hex(text);
  exe->json = to_json(*c.main, &c.stats);
  exe->plan = std::move(c.plan);
  for (const Type& t : exe->plan->result_types()) {
    exe->out_types.push_back(to_pjrt(t.dtype));
    exe->out_dim_sizes.push_back(t.dims.size());
    exe->out_dims.insert(exe->out_dims.end(), t.dims.begin(), t.dims.end());
    exe->mem_kinds.push_back(kMemoryKind);
    exe->mem_kind_sizes.push_back(std::strlen(kMemoryKind));
  }
  static const char* kFlops = "flops";
  PJRT_NamedValue nv;
  std::memset(&nv, 0, sizeof nv);
  nv.struct_size = sizeof nv;
  nv.name = kFlops;
  nv.name_size = std::strlen(kFlops);
  nv.type = PJRT_NamedValue_kFloat;
  nv.float_value = (float)exe->plan->total_flops();
  nv.value_size = 1;
  exe->cost.push_back(nv);
  auto* le = new PJRT_LoadedExecutable();
  le->exe = exe;
  le->client = client;
  *out = le;
  return nullptr;
}

PJRT_Error* Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* args) {
  CHECK_ARGS(PJRT_Client_DefaultDeviceAssignment_Args, default_assignment);
  size_t n = (size_t)args->num_replicas * args->num_partitions;
  if (args->default_assignment_size < n)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "default_assignment buffer too small");
  const int nd = (int)args->client->device_ptrs.size();
  for (size_t i = 0; i < n; ++i) args->default_assignment[i] = (int)(i % (size_t)nd);
  return nullptr;
}

PJRT_Device* pick_device(PJRT_Client* c, PJRT_Device* d, PJRT_Memory* m) {
  if (d) return d;
  if (m && !m->devices.empty()) return m->devices[0];
  return c->device_ptrs.at(0);
}

PJRT_Buffer* new_buffer(PJRT_Client* c, PJRT_Device* d, const mfxp::Type& t, PJRT_Error** err) {
  hipError_t e;
  size_t bytes = (size_t)t.bytes();
  void* p = c->alloc(d->ordinal, bytes, e);
  if (!p) {
    *err = hip_error(e, "hipMalloc");
    return nullptr;
  }
  auto* b = new PJRT_Buffer();
  b->client = c;
  b->device = d;
  b->ptr = p;
  b->bytes = bytes;
  b->type = t;
  return b;
}

// Dense row-major copy of a host array given (optional) byte strides.
const void* pack_host(const void* data, const mfxp::Type& t, const int64_t* bs, size_t nbs,
                      std::vector<uint8_t>& tmp) {
  if (!bs || nbs == 0) return data;
  const int r = t.rank();
  if ((int)nbs != r) return nullptr;
  const int eb = dtype_bytes(t.dtype);
  auto cs = contiguous_strides(t.dims);
  bool dense = true;
  for (int i = 0; i < r; ++i)
    if (t.dims[i] > 1 && bs[i] != cs[i] * eb) dense = false;
  if (dense) return data;
  tmp.resize((size_t)t.bytes());
  const int64_t n = t.numel();
  std::vector<int64_t> idx(r, 0);
  for (int64_t k = 0; k < n; ++k) {
    int64_t off = 0;
    for (int i = 0; i < r; ++i) off += idx[i] * bs[i];
    std::memcpy(tmp.data() + k * eb, (const uint8_t*)data + off, eb);
    for (int i = r - 1; i >= 0; --i) {
      if (++idx[i] < t.dims[i]) break;
      idx[i] = 0;
    }
  }
  return tmp.data();
}

PJRT_Error* Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* args) {
  CHECK_ARGS(PJRT_Client_BufferFromHostBuffer_Args, buffer);
  GUARD_BEGIN
  mfxp::Type t;
  t.dtype = from_pjrt(args->type);
  if (t.dtype == DType::kInvalid || dtype_bytes(t.dtype) == 0)
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "BufferFromHostBuffer: unsupported element type " +
                                                         std::to_string((int)args->type));
  t.dims.assign(args->dims, args->dims + args->num_dims);
  for (int64_t d : t.dims)
    if (d < 0) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "negative dimension");
  if (args->device_layout && args->device_layout->type != PJRT_Buffer_MemoryLayout_Type_Tiled)
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "BufferFromHostBuffer: strided device layouts");
  std::vector<uint8_t> tmp;
  const void* src = pack_host(args->data, t, args->byte_strides, args->num_byte_strides, tmp);
  if (!src) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "byte_strides rank does not match dims");
  PJRT_Device* d = pick_device(args->client, args->device, args->memory);
  PJRT_Error* err = nullptr;
  PJRT_Buffer* b = new_buffer(args->client, d, t, &err);
  if (!b) return err;
  hipError_t e = hipSetDevice(d->ordinal);
  if (e == hipSuccess && b->bytes)
    e = hipMemcpyAsync(b->ptr, src, b->bytes, hipMemcpyHostToDevice, d->stream);
  // The host data may be released as soon as we return: wait for the copy.
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  if (e != hipSuccess) {
    b->free_memory();
    delete b;
    return hip_error(e, "host-to-device copy");
  }
  b->ready = std::make_shared<EventState>();
  args->buffer = b;
  args->done_with_host_buffer = new PJRT_Event{std::make_shared<EventState>()};
  return nullptr;
  GUARD_END
}

PJRT_Error* Client_CreateViewOfDeviceBuffer(PJRT_Client_CreateViewOfDeviceBuffer_Args* args) {
  CHECK_ARGS(PJRT_Client_CreateViewOfDeviceBuffer_Args, buffer);
  GUARD_BEGIN
  mfxp::Type t;
  t.dtype = from_pjrt(args->element_type);
  if (t.dtype == DType::kInvalid) return make_error(PJRT_Error_Code_UNIMPLEMENTED, "unsupported element type");
  t.dims.assign(args->dims, args->dims + args->num_dims);
  if (args->layout && args->layout->type != PJRT_Buffer_MemoryLayout_Type_Tiled)
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "CreateViewOfDeviceBuffer: strided layouts");
  PJRT_Device* dev = pick_device(args->client, args->device, nullptr);
  // The memory is ready once the work enqueued so far on the producer's
  // stream (`stream`, or the legacy null stream when none is given) is done:
  // the plugin's stream waits for it there before anything reads the view.
  {
    hipError_t e = hipSetDevice(dev->ordinal);
    hipEvent_t ev = nullptr;
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(ev, reinterpret_cast<hipStream_t>(args->stream));
    if (e == hipSuccess) e = hipStreamWaitEvent(dev->stream, ev, 0);
    if (ev) (void)hipEventDestroy(ev);
    if (e != hipSuccess) return hip_error(e, "CreateViewOfDeviceBuffer: ordering after the producer's stream");
  }
  auto* b = new PJRT_Buffer();
  b->client = args->client;
  b->device = dev;
  b->ptr = args->device_buffer_ptr;
  b->bytes = (size_t)t.bytes();
  b->type = t;
  b->owned = false;
  b->on_delete = args->on_delete_callback;
  b->on_delete_arg = args->on_delete_callback_arg;
  b->ready = std::make_shared<EventState>();
  args->buffer = b;
  return nullptr;
  GUARD_END
}

PJRT_Error* Client_CreateUninitializedBuffer(PJRT_Client_CreateUninitializedBuffer_Args* args) {
  CHECK_ARGS(PJRT_Client_CreateUninitializedBuffer_Args, buffer);
  GUARD_BEGIN
  mfxp::Type t;
  t.dtype = from_pjrt(args->shape_element_type);
  if (t.dtype == DType::kInvalid) return make_error(PJRT_Error_Code_UNIMPLEMENTED, "unsupported element type");
  t.dims.assign(args->shape_dims, args->shape_dims + args->shape_num_dims);
  PJRT_Error* err = nullptr;
  PJRT_Buffer* b = new_buffer(args->client, pick_device(args->client, args->device, args->memory), t, &err);
  if (!b) return err;
  b->ready = std::make_shared<EventState>();
  args->buffer = b;
  return nullptr;
  GUARD_END
}

// ---------------------------------------------------------------------------
// Device descriptions, devices, memories, topology

PJRT_Error* DeviceDescription_Id(PJRT_DeviceDescription_Id_Args* args) {
  CHECK_ARGS(PJRT_DeviceDescription_Id_Args, id);
  args->id = args->device_description->id;
  return nullptr;
}
PJRT_Error* DeviceDescription_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* args) {
  CHECK_ARGS(PJRT_DeviceDescription_ProcessIndex_Args, process_index);
  args->process_index = 0;
  return nullptr;
}
PJRT_Error* DeviceDescription_Attributes(PJRT_DeviceDescription_Attributes_Args* args) {
  CHECK_ARGS(PJRT_DeviceDescription_Attributes_Args, attributes);
  args->num_attributes = args->device_description->attrs.size();
  args->attributes = args->device_description->attrs.data();
  return nullptr;
}
PJRT_Error* DeviceDescription_Kind(PJRT_DeviceDescription_Kind_Args* args) {
  CHECK_ARGS(PJRT_DeviceDescription_Kind_Args, device_kind_size);
  args->device_kind = args->device_description->kind.c_str();
  args->device_kind_size = args->device_description->kind.size();
  return nullptr;
}
PJRT_Error* DeviceDescription_DebugString(PJRT_DeviceDescription_DebugString_Args* args) {
  CHECK_ARGS(PJRT_DeviceDescription_DebugString_Args, debug_string_size);
  args->debug_string = args->device_description->debug.c_str();
  args->debug_string_size = args->device_description->debug.size();
  return nullptr;
}
PJRT_Error* DeviceDescription_ToString(PJRT_DeviceDescription_ToString_Args* args) {
  CHECK_ARGS(PJRT_DeviceDescription_ToString_Args, to_string_size);
  args->to_string = args->device_description->tostr.c_str();
  args->to_string_size = args->device_description->tostr.size();
  return nullptr;
}

PJRT_Error* Device_GetDescription(PJRT_Device_GetDescription_Args* args) {
  CHECK_ARGS(PJRT_Device_GetDescription_Args, device_description);
  args->device_description = &args->device->desc;
  return nullptr;
}
PJRT_Error* Device_IsAddressable(PJRT_Device_IsAddressable_Args* args) {
  CHECK_ARGS(PJRT_Device_IsAddressable_Args, is_addressable);
  args->is_addressable = true;
  return nullptr;
}
PJRT_Error* Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* args) {
  CHECK_ARGS(PJRT_Device_LocalHardwareId_Args, local_hardware_id);
  args->local_hardware_id = args->device->ordinal;
  return nullptr;
}
PJRT_Error* Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* args) {
  CHECK_ARGS(PJRT_Device_AddressableMemories_Args, num_memories);
  args->memories = &args->device->memory;
  args->num_memories = 1;
  return nullptr;
}
PJRT_Error* Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* args) {
  CHECK_ARGS(PJRT_Device_DefaultMemory_Args, memory);
  args->memory = args->device->memory;
  return nullptr;
}
PJRT_Error* Device_MemoryStats(PJRT_Device_MemoryStats_Args* args) {
  CHECK_ARGS(PJRT_Device_MemoryStats_Args, bytes_in_use);
  size_t free_b = 0, total_b = 0;
  hipError_t e = hipSetDevice(args->device->ordinal);
  if (e == hipSuccess) e = hipMemGetInfo(&free_b, &total_b);
  if (e != hipSuccess) return hip_error(e, "hipMemGetInfo");
  args->bytes_in_use = (int64_t)(total_b - free_b);
  if (args->struct_size >= PJRT_ABI_SIZE(PJRT_Device_MemoryStats_Args, bytes_limit_is_set)) {
    args->peak_bytes_in_use_is_set = false;
    args->num_allocs_is_set = false;
    args->largest_alloc_size_is_set = false;
    args->bytes_limit = (int64_t)total_b;
    args->bytes_limit_is_set = true;
  }
  return nullptr;
}

PJRT_Error* Memory_Id(PJRT_Memory_Id_Args* args) {
  CHECK_ARGS(PJRT_Memory_Id_Args, id);
  args->id = args->memory->id;
  return nullptr;
}
PJRT_Error* Memory_Kind(PJRT_Memory_Kind_Args* args) {
  CHECK_ARGS(PJRT_Memory_Kind_Args, kind_size);
  args->kind = args->memory->kind.c_str();
  args->kind_size = args->memory->kind.size();
  return nullptr;
}
PJRT_Error* Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* args) {
  CHECK_ARGS(PJRT_Memory_Kind_Id_Args, kind_id);
  args->kind_id = 0;
  return nullptr;
}
PJRT_Error* Memory_DebugString(PJRT_Memory_DebugString_Args* args) {
  CHECK_ARGS(PJRT_Memory_DebugString_Args, debug_string_size);
  args->debug_string = args->memory->debug.c_str();
  args->debug_string_size = args->memory->debug.size();
  return nullptr;
}
PJRT_Error* Memory_ToString(PJRT_Memory_ToString_Args* args) {
  CHECK_ARGS(PJRT_Memory_ToString_Args, to_string_size);
  args->to_string = args->memory->tostr.c_str();
  args->to_string_size = args->memory->tostr.size();
  return nullptr;
}
PJRT_Error* Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* args) {
  CHECK_ARGS(PJRT_Memory_AddressableByDevices_Args, num_devices);
  args->devices = args->memory->devices.data();
  args->num_devices = args->memory->devices.size();
  return nullptr;
}

PJRT_Error* TopologyDescription_Destroy(PJRT_TopologyDescription_Destroy_Args* args) {
  return nullptr;  // owned by its client
}
PJRT_Error* TopologyDescription_PlatformName(PJRT_TopologyDescription_PlatformName_Args* args) {
  CHECK_ARGS(PJRT_TopologyDescription_PlatformName_Args, platform_name_size);
  const std::string& n = args->topology->client->platform_name;
  args->platform_name = n.c_str();
  args->platform_name_size = n.size();
  return nullptr;
}
PJRT_Error* TopologyDescription_PlatformVersion(PJRT_TopologyDescription_PlatformVersion_Args* args) {
  CHECK_ARGS(PJRT_TopologyDescription_PlatformVersion_Args, platform_version_size);
  const std::string& n = args->topology->client->platform_version;
  args->platform_version = n.c_str();
  args->platform_version_size = n.size();
  return nullptr;
}
PJRT_Error* TopologyDescription_GetDeviceDescriptions(PJRT_TopologyDescription_GetDeviceDescriptions_Args* args) {
  CHECK_ARGS(PJRT_TopologyDescription_GetDeviceDescriptions_Args, num_descriptions);
  args->descriptions = args->topology->descs.data();
  args->num_descriptions = args->topology->descs.size();
  return nullptr;
}
PJRT_Error* TopologyDescription_Attributes(PJRT_TopologyDescription_Attributes_Args* args) {
  CHECK_ARGS(PJRT_TopologyDescription_Attributes_Args, num_attributes);
  args->attributes = nullptr;
  args->num_attributes = 0;
  return nullptr;
}

// ---------------------------------------------------------------------------
// Executables

PJRT_Error* Executable_Destroy(PJRT_Executable_Destroy_Args* args) {
  CHECK_ARGS(PJRT_Executable_Destroy_Args, executable);
  if (args->executable) args->executable->unref();
  return nullptr;
}
PJRT_Error* Executable_Name(PJRT_Executable_Name_Args* args) {
  CHECK_ARGS(PJRT_Executable_Name_Args, executable_name_size);
  args->executable_name = args->executable->name.c_str();
  args->executable_name_size = args->executable->name.size();
  return nullptr;
}
PJRT_Error* Executable_NumReplicas(PJRT_Executable_NumReplicas_Args* args) {
  CHECK_ARGS(PJRT_Executable_NumReplicas_Args, num_replicas);
  args->num_replicas = 1;
  return nullptr;
}
PJRT_Error* Executable_NumPartitions(PJRT_Executable_NumPartitions_Args* args) {
  CHECK_ARGS(PJRT_Executable_NumPartitions_Args, num_partitions);
  args->num_partitions = 1;
  return nullptr;
}
PJRT_Error* Executable_NumOutputs(PJRT_Executable_NumOutputs_Args* args) {
  CHECK_ARGS(PJRT_Executable_NumOutputs_Args, num_outputs);
  args->num_outputs = args->executable->out_types.size();
  return nullptr;
}
PJRT_Error* Executable_SizeOfGeneratedCodeInBytes(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* args) {
  CHECK_ARGS(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args, size_in_bytes);
  args->size_in_bytes = 0;
  return nullptr;
}
PJRT_Error* Executable_GetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* args) {
  CHECK_ARGS(PJRT_Executable_GetCostAnalysis_Args, properties);
  args->num_properties = args->executable->cost.size();
  args->properties = args->executable->cost.data();
  return nullptr;
}
PJRT_Error* Executable_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* args) {
  CHECK_ARGS(PJRT_Executable_OutputMemoryKinds_Args, memory_kind_sizes);
  args->num_outputs = args->executable->mem_kinds.size();
  args->memory_kinds = args->executable->mem_kinds.data();
  args->memory_kind_sizes = args->executable->mem_kind_sizes.data();
  return nullptr;
}
PJRT_Error* Executable_OptimizedProgram(PJRT_Executable_OptimizedProgram_Args* args) {
  return unimplemented("PJRT_Executable_OptimizedProgram");
}
// Serialized executable: the magic kSerialMagic, a format version, the text
// length (little-endian u32, u64) and the module text.  The plan is rebuilt
// from the text on load (same parser, rewriter and planner, so the same
// launches), which makes the blob independent of device addresses and of the
// hipRTC code objects cached per process.  (The reference returns an empty
// blob, src/jax_mlx_pjrt.cpp:1585-1601.)
constexpr char kSerialMagic[8] = {'M', 'F', 'X', 'P', 'J', 'R', 'T', '\n'};
constexpr uint32_t kSerialVersion = 1;
constexpr size_t kSerialHeader = sizeof kSerialMagic + 4 + 8;

void delete_serialized(PJRT_SerializedExecutable* p) { delete reinterpret_cast<std::string*>(p); }

PJRT_Error* Executable_Serialize(PJRT_Executable_Serialize_Args* args) {
  CHECK_ARGS(PJRT_Executable_Serialize_Args, serialized_executable_deleter);
  if (!args->executable) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Serialize: no executable");
  const std::string& text = args->executable->text;
  auto* blob = new std::string(kSerialMagic, sizeof kSerialMagic);
  const uint64_t n = text.size();
  for (int i = 0; i < 4; ++i) blob->push_back((char)((kSerialVersion >> (8 * i)) & 0xff));
  for (int i = 0; i < 8; ++i) blob->push_back((char)((n >> (8 * i)) & 0xff));
  blob->append(text);
  args->serialized_bytes = blob->data();
  args->serialized_bytes_size = blob->size();
  args->serialized_executable = reinterpret_cast<PJRT_SerializedExecutable*>(blob);
  args->serialized_executable_deleter = delete_serialized;
  return nullptr;
}

PJRT_Error* Executable_DeserializeAndLoad(PJRT_Executable_DeserializeAndLoad_Args* args) {
  CHECK_ARGS(PJRT_Executable_DeserializeAndLoad_Args, loaded_executable);
  GUARD_BEGIN
  if (!args->client) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "DeserializeAndLoad: no client");
  const char* b = args->serialized_executable;
  const size_t size = b ? args->serialized_executable_size : 0;
  if (size < kSerialHeader || std::memcmp(b, kSerialMagic, sizeof kSerialMagic) != 0)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT,
                      "DeserializeAndLoad: not an executable serialized by this plugin");
  uint32_t version = 0;
  uint64_t n = 0;
  for (int i = 0; i < 4; ++i) version |= (uint32_t)(unsigned char)b[sizeof kSerialMagic + i] << (8 * i);
  for (int i = 0; i < 8; ++i) n |= (uint64_t)(unsigned char)b[sizeof kSerialMagic + 4 + i] << (8 * i);
  if (version != kSerialVersion)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT,
                      "DeserializeAndLoad: serialized format version " + std::to_string(version) +
                          ", this plugin reads version " + std::to_string(kSerialVersion));
  if (n != size - kSerialHeader)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "DeserializeAndLoad: truncated or padded executable");
  return load_text(args->client, std::string(b + kSerialHeader, (size_t)n), &args->loaded_executable);
  GUARD_END
}
PJRT_Error* Executable_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* args) {
  CHECK_ARGS(PJRT_Executable_OutputElementTypes_Args, num_output_types);
  args->output_types = args->executable->out_types.data();
  args->num_output_types = args->executable->out_types.size();
  return nullptr;
}
PJRT_Error* Executable_OutputDimensions(PJRT_Executable_OutputDimensions_Args* args) {
  CHECK_ARGS(PJRT_Executable_OutputDimensions_Args, dim_sizes);
  args->num_outputs = args->executable->out_dim_sizes.size();
  args->dims = args->executable->out_dims.data();
  args->dim_sizes = args->executable->out_dim_sizes.data();
  return nullptr;
}
PJRT_Error* Executable_Fingerprint(PJRT_Executable_Fingerprint_Args* args) {
  CHECK_ARGS(PJRT_Executable_Fingerprint_Args, executable_fingerprint_size);
  args->executable_fingerprint = args->executable->fingerprint.c_str();
  args->executable_fingerprint_size = args->executable->fingerprint.size();
  return nullptr;
}
PJRT_Error* Executable_GetCompiledMemoryStats(PJRT_Executable_GetCompiledMemoryStats_Args* args) {
  CHECK_ARGS(PJRT_Executable_GetCompiledMemoryStats_Args, total_size_in_bytes);
  const Plan& p = *args->executable->plan;
  int64_t arg_b = 0, out_b = 0;
  for (const Type& t : p.param_types()) arg_b += t.bytes();
  for (const Type& t : p.result_types()) out_b += t.bytes();
  args->generated_code_size_in_bytes = 0;
  args->argument_size_in_bytes = arg_b;
  args->output_size_in_bytes = out_b;
  args->alias_size_in_bytes = 0;
  args->temp_size_in_bytes = (int64_t)p.arena_bytes();
  args->host_generated_code_size_in_bytes = 0;
  args->host_argument_size_in_bytes = 0;
  args->host_output_size_in_bytes = 0;
  args->host_alias_size_in_bytes = 0;
  args->host_temp_size_in_bytes = 0;
  args->peak_memory_in_bytes = arg_b + out_b + (int64_t)p.arena_bytes();
  args->total_size_in_bytes = args->peak_memory_in_bytes;
  return nullptr;
}

PJRT_Error* LoadedExecutable_Destroy(PJRT_LoadedExecutable_Destroy_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_Destroy_Args, executable);
  if (args->executable) {
    args->executable->exe->unref();
    delete args->executable;
  }
  return nullptr;
}
PJRT_Error* LoadedExecutable_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_GetExecutable_Args, executable);
  args->loaded_executable->exe->refs++;
  args->executable = args->loaded_executable->exe;
  return nullptr;
}
PJRT_Error* LoadedExecutable_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_AddressableDevices_Args, num_addressable_devices);
  args->addressable_devices = args->executable->client->device_ptrs.data();
  args->num_addressable_devices = 1;
  return nullptr;
}
PJRT_Error* LoadedExecutable_Delete(PJRT_LoadedExecutable_Delete_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_Delete_Args, executable);
  args->executable->deleted = true;
  return nullptr;
}
PJRT_Error* LoadedExecutable_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_IsDeleted_Args, is_deleted);
  args->is_deleted = args->executable->deleted;
  return nullptr;
}
PJRT_Error* LoadedExecutable_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_Fingerprint_Args, executable_fingerprint_size);
  args->executable_fingerprint = args->executable->exe->fingerprint.c_str();
  args->executable_fingerprint_size = args->executable->exe->fingerprint.size();
  return nullptr;
}

struct SerializedAssignment {
  std::string bytes;
};

void delete_assignment(PJRT_DeviceAssignmentSerialized* p) {
  delete reinterpret_cast<SerializedAssignment*>(p);
}

PJRT_Error* LoadedExecutable_GetDeviceAssignment(PJRT_LoadedExecutable_GetDeviceAssignment_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_GetDeviceAssignment_Args, serialized_device_assignment_deleter);
  // DeviceAssignmentProto{replica_count: 1, computation_count: 1,
  //   computation_devices: [{replica_device_ids: [0]}]} in protobuf wire format.
  auto* s = new SerializedAssignment{std::string("\x08\x01\x10\x01\x1a\x02\x08\x00", 8)};
  args->serialized_bytes = s->bytes.data();
  args->serialized_bytes_size = s->bytes.size();
  args->serialized_device_assignment = reinterpret_cast<PJRT_DeviceAssignmentSerialized*>(s);
  args->serialized_device_assignment_deleter = delete_assignment;
  return nullptr;
}

PJRT_Error* LoadedExecutable_Execute(PJRT_LoadedExecutable_Execute_Args* args) {
  CHECK_ARGS(PJRT_LoadedExecutable_Execute_Args, device_complete_events);
  GUARD_BEGIN
  PJRT_LoadedExecutable* le = args->executable;
  if (le->deleted) return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "Execute: executable was deleted");
  if (args->num_devices != 1)
    return make_error(PJRT_Error_Code_UNIMPLEMENTED, "Execute: one device per call (got " +
                                                         std::to_string(args->num_devices) + ")");
  Plan& plan = *le->exe->plan;
  const auto& pt = plan.param_types();
  if (args->num_args != pt.size())
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: expected " + std::to_string(pt.size()) +
                                                            " arguments, got " + std::to_string(args->num_args));
  PJRT_Client* c = le->client;
  PJRT_Device* dev = c->device_ptrs.at(0);
  if (args->struct_size >= PJRT_ABI_SIZE(PJRT_LoadedExecutable_Execute_Args, execute_device) &&
      args->execute_device)
    dev = args->execute_device;
  ExecBuffers b;
  b.stream = dev->stream;
  for (size_t i = 0; i < args->num_args; ++i) {
    PJRT_Buffer* in = args->argument_lists[0][i];
    if (!in || in->deleted)
      return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: argument " + std::to_string(i) + " is deleted");
    if (in->type != pt[i])
      return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: argument " + std::to_string(i) + " is " +
                                                              in->type.str() + ", the module expects " + pt[i].str());
    if (in->device != dev)
      return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "Execute: argument on another device");
    b.params.push_back(in->ptr);
  }
  hipError_t e = hipSetDevice(dev->ordinal);
  if (e != hipSuccess) return hip_error(e, "hipSetDevice");
  std::vector<PJRT_Buffer*> outs;
  PJRT_Error* err = nullptr;
  for (const Type& t : plan.result_types()) {
    PJRT_Buffer* o = new_buffer(c, dev, t, &err);
    if (!o) {
      for (PJRT_Buffer* x : outs) {
        x->free_memory();
        delete x;
      }
      return err;
    }
    outs.push_back(o);
    b.outputs.push_back(o->ptr);
  }
  std::string msg;
  int rc = plan.run(b, msg);
  if (rc != MFX_OK) {
    (void)hipStreamSynchronize(dev->stream);
    for (PJRT_Buffer* x : outs) {
      x->free_memory();
      delete x;
    }
    return make_error(PJRT_Error_Code_INTERNAL, "Execute: " + msg);
  }
  auto st = record_event(dev->stream, &err);
  if (err) return err;
  for (size_t j = 0; j < outs.size(); ++j) {
    outs[j]->ready = st;
    args->output_lists[0][j] = outs[j];
  }
  if (args->device_complete_events) args->device_complete_events[0] = new PJRT_Event{st};
  return nullptr;
  GUARD_END
}

// ---------------------------------------------------------------------------
// Buffers

PJRT_Error* Buffer_Destroy(PJRT_Buffer_Destroy_Args* args) {
  CHECK_ARGS(PJRT_Buffer_Destroy_Args, buffer);
  if (!args->buffer) return nullptr;
  PJRT_Buffer* b = args->buffer;
  b->free_memory();
  {
    std::lock_guard<std::mutex> g(b->mu);
    if (b->release_pending) {
      b->destroyed = true;  // freed by the last DecreaseExternalReferenceCount
      return nullptr;
    }
  }
  delete b;
  return nullptr;
}
PJRT_Error* Buffer_ElementType(PJRT_Buffer_ElementType_Args* args) {
  CHECK_ARGS(PJRT_Buffer_ElementType_Args, type);
  args->type = to_pjrt(args->buffer->type.dtype);
  return nullptr;
}
PJRT_Error* Buffer_Dimensions(PJRT_Buffer_Dimensions_Args* args) {
  CHECK_ARGS(PJRT_Buffer_Dimensions_Args, num_dims);
  args->dims = args->buffer->type.dims.data();
  args->num_dims = args->buffer->type.dims.size();
  return nullptr;
}
PJRT_Error* Buffer_UnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* args) {
  CHECK_ARGS(PJRT_Buffer_UnpaddedDimensions_Args, num_dims);
  args->unpadded_dims = args->buffer->type.dims.data();
  args->num_dims = args->buffer->type.dims.size();
  return nullptr;
}
PJRT_Error* Buffer_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* args) {
  CHECK_ARGS(PJRT_Buffer_DynamicDimensionIndices_Args, num_dynamic_dims);
  args->dynamic_dim_indices = nullptr;
  args->num_dynamic_dims = 0;
  return nullptr;
}
PJRT_Error* Buffer_GetMemoryLayout(PJRT_Buffer_GetMemoryLayout_Args* args) {
  CHECK_ARGS(PJRT_Buffer_GetMemoryLayout_Args, layout);
  PJRT_Buffer* b = args->buffer;
  const int r = b->type.rank();
  b->minor_to_major.resize(r);
  for (int i = 0; i < r; ++i) b->minor_to_major[i] = r - 1 - i;
  std::memset(&args->layout, 0, sizeof args->layout);
  args->layout.struct_size = sizeof(PJRT_Buffer_MemoryLayout);
  args->layout.type = PJRT_Buffer_MemoryLayout_Type_Tiled;
  args->layout.tiled.struct_size = sizeof(PJRT_Buffer_MemoryLayout_Tiled);
  args->layout.tiled.minor_to_major = b->minor_to_major.data();
  args->layout.tiled.minor_to_major_size = r;
  args->layout.tiled.num_tiles = 0;
  return nullptr;
}
PJRT_Error* Buffer_OnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* args) {
  CHECK_ARGS(PJRT_Buffer_OnDeviceSizeInBytes_Args, on_device_size_in_bytes);
  args->on_device_size_in_bytes = args->buffer->bytes;
  return nullptr;
}
PJRT_Error* Buffer_Device(PJRT_Buffer_Device_Args* args) {
  CHECK_ARGS(PJRT_Buffer_Device_Args, device);
  args->device = args->buffer->device;
  return nullptr;
}
PJRT_Error* Buffer_Memory(PJRT_Buffer_Memory_Args* args) {
  CHECK_ARGS(PJRT_Buffer_Memory_Args, memory);
  args->memory = args->buffer->device->memory;
  return nullptr;
}
PJRT_Error* Buffer_Delete(PJRT_Buffer_Delete_Args* args) {
  CHECK_ARGS(PJRT_Buffer_Delete_Args, buffer);
  args->buffer->free_memory();
  return nullptr;
}
PJRT_Error* Buffer_IsDeleted(PJRT_Buffer_IsDeleted_Args* args) {
  CHECK_ARGS(PJRT_Buffer_IsDeleted_Args, is_deleted);
  args->is_deleted = args->buffer->deleted;
  return nullptr;
}
PJRT_Error* copy_buffer(PJRT_Buffer* src, PJRT_Device* dst_dev, PJRT_Buffer** out) {
  if (src->deleted) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "copy of a deleted buffer");
  PJRT_Error* err = nullptr;
  PJRT_Buffer* b = new_buffer(src->client, dst_dev, src->type, &err);
  if (!b) return err;
  hipError_t e = hipSetDevice(dst_dev->ordinal);
  if (e == hipSuccess && b->bytes) {
    if (src->device == dst_dev)
      e = hipMemcpyAsync(b->ptr, src->ptr, b->bytes, hipMemcpyDeviceToDevice, dst_dev->stream);
    else
      e = hipMemcpyPeerAsync(b->ptr, dst_dev->ordinal, src->ptr, src->device->ordinal, b->bytes, dst_dev->stream);
  }
  if (e != hipSuccess) {
    b->free_memory();
    delete b;
    return hip_error(e, "buffer copy");
  }
  b->ready = record_event(dst_dev->stream, &err);
  *out = b;
  return err;
}
PJRT_Error* Buffer_CopyToDevice(PJRT_Buffer_CopyToDevice_Args* args) {
  CHECK_ARGS(PJRT_Buffer_CopyToDevice_Args, dst_buffer);
  GUARD_BEGIN
  return copy_buffer(args->buffer, args->dst_device, &args->dst_buffer);
  GUARD_END
}
PJRT_Error* Buffer_CopyToMemory(PJRT_Buffer_CopyToMemory_Args* args) {
  CHECK_ARGS(PJRT_Buffer_CopyToMemory_Args, dst_buffer);
  GUARD_BEGIN
  PJRT_Device* d = args->dst_memory && !args->dst_memory->devices.empty() ? args->dst_memory->devices[0]
                                                                          : args->buffer->device;
  return copy_buffer(args->buffer, d, &args->dst_buffer);
  GUARD_END
}
PJRT_Error* Buffer_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* args) {
  CHECK_ARGS(PJRT_Buffer_ToHostBuffer_Args, event);
  GUARD_BEGIN
  PJRT_Buffer* b = args->src;
  if (b->deleted) return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "ToHostBuffer of a deleted buffer");
  if (args->host_layout) {
    const PJRT_Buffer_MemoryLayout* hl = args->host_layout;
    bool row_major = hl->type == PJRT_Buffer_MemoryLayout_Type_Tiled && hl->tiled.num_tiles == 0;
    if (row_major && hl->tiled.minor_to_major) {
      const int r = b->type.rank();
      for (int i = 0; i < (int)hl->tiled.minor_to_major_size && i < r; ++i)
        row_major &= hl->tiled.minor_to_major[i] == r - 1 - i;
    }
    if (!row_major) return make_error(PJRT_Error_Code_UNIMPLEMENTED, "ToHostBuffer: non row-major host layouts");
  }
  if (!args->dst) {
    args->dst_size = b->bytes;
    return nullptr;
  }
  if (args->dst_size < b->bytes)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "ToHostBuffer: destination too small");
  PJRT_Device* d = b->device;
  hipError_t e = hipSetDevice(d->ordinal);
  if (e == hipSuccess && b->bytes) e = hipMemcpyAsync(args->dst, b->ptr, b->bytes, hipMemcpyDeviceToHost, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  if (e != hipSuccess) return hip_error(e, "device-to-host copy");
  args->event = new PJRT_Event{std::make_shared<EventState>()};
  return nullptr;
  GUARD_END
}
PJRT_Error* Buffer_CopyRawToHost(PJRT_Buffer_CopyRawToHost_Args* args) {
  CHECK_ARGS(PJRT_Buffer_CopyRawToHost_Args, event);
  GUARD_BEGIN
  PJRT_Buffer* b = args->buffer;
  if (args->offset < 0 || args->transfer_size < 0 || (size_t)(args->offset + args->transfer_size) > b->bytes)
    return make_error(PJRT_Error_Code_INVALID_ARGUMENT, "CopyRawToHost: range outside the buffer");
  PJRT_Device* d = b->device;
  hipError_t e = hipSetDevice(d->ordinal);
  if (e == hipSuccess && args->transfer_size)
    e = hipMemcpyAsync(args->dst, (char*)b->ptr + args->offset, args->transfer_size, hipMemcpyDeviceToHost, d->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
  if (e != hipSuccess) return hip_error(e, "device-to-host copy");
  args->event = new PJRT_Event{std::make_shared<EventState>()};
  return nullptr;
  GUARD_END
}
PJRT_Error* Buffer_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* args) {
  CHECK_ARGS(PJRT_Buffer_IsOnCpu_Args, is_on_cpu);
  args->is_on_cpu = false;
  return nullptr;
}
PJRT_Error* Buffer_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* args) {
  CHECK_ARGS(PJRT_Buffer_ReadyEvent_Args, event);
  auto st = args->buffer->ready ? args->buffer->ready : std::make_shared<EventState>();
  args->event = new PJRT_Event{st};
  return nullptr;
}
PJRT_Error* Buffer_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* args) {
  CHECK_ARGS(PJRT_Buffer_UnsafePointer_Args, buffer_pointer);
  args->buffer_pointer = (uintptr_t)args->buffer->ptr;
  return nullptr;
}
PJRT_Error* Buffer_IncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* args) {
  CHECK_ARGS(PJRT_Buffer_IncreaseExternalReferenceCount_Args, buffer);
  std::lock_guard<std::mutex> g(args->buffer->mu);
  if (args->buffer->deleted)
    return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "external reference to a deleted buffer");
  args->buffer->ext_refs++;
  return nullptr;
}
PJRT_Error* Buffer_DecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* args) {
  CHECK_ARGS(PJRT_Buffer_DecreaseExternalReferenceCount_Args, buffer);
  PJRT_Buffer* b = args->buffer;
  bool destroy = false;
  {
    std::lock_guard<std::mutex> g(b->mu);
    if (b->ext_refs.load() <= 0)
      return make_error(PJRT_Error_Code_FAILED_PRECONDITION, "external reference count is already zero");
    if (--b->ext_refs == 0 && b->release_pending) {
      b->release_locked();
      destroy = b->destroyed;
    }
  }
  if (destroy) delete b;
  return nullptr;
}
PJRT_Error* Buffer_OpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* args) {
  CHECK_ARGS(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args, device_memory_ptr);
  args->device_memory_ptr = args->buffer->ptr;
  return nullptr;
}

PJRT_Error* ExecuteContext_Create(PJRT_ExecuteContext_Create_Args* args) {
  CHECK_ARGS(PJRT_ExecuteContext_Create_Args, context);
  args->context = new PJRT_ExecuteContext();
  return nullptr;
}
PJRT_Error* ExecuteContext_Destroy(PJRT_ExecuteContext_Destroy_Args* args) {
  CHECK_ARGS(PJRT_ExecuteContext_Destroy_Args, context);
  delete args->context;
  return nullptr;
}

// Generic answer for the slots this plugin does not provide.
#define STUB_FN(name)                                      \
  PJRT_Error* Stub_##name(void*) { return unimplemented("PJRT_" #name); }
STUB_FN(CopyToDeviceStream_Destroy)
STUB_FN(CopyToDeviceStream_AddChunk)
STUB_FN(CopyToDeviceStream_TotalBytes)
STUB_FN(CopyToDeviceStream_GranuleSize)
STUB_FN(CopyToDeviceStream_CurrentBytes)
STUB_FN(TopologyDescription_Create)
STUB_FN(TopologyDescription_Serialize)
STUB_FN(Compile)
STUB_FN(AsyncHostToDeviceTransferManager_Destroy)
STUB_FN(AsyncHostToDeviceTransferManager_TransferData)
STUB_FN(Client_CreateBuffersForAsyncHostToDevice)
STUB_FN(AsyncHostToDeviceTransferManager_RetrieveBuffer)
STUB_FN(AsyncHostToDeviceTransferManager_Device)
STUB_FN(AsyncHostToDeviceTransferManager_BufferCount)
STUB_FN(AsyncHostToDeviceTransferManager_BufferSize)
STUB_FN(AsyncHostToDeviceTransferManager_SetBufferError)
STUB_FN(AsyncHostToDeviceTransferManager_AddMetadata)
STUB_FN(Client_DmaMap)
STUB_FN(Client_DmaUnmap)
STUB_FN(Client_UpdateGlobalProcessInfo)
STUB_FN(TopologyDescription_Deserialize)
STUB_FN(Client_CreateAliasBuffer)
STUB_FN(Client_FulfillAliasBuffer)
STUB_FN(Client_CreateErrorBuffer)
STUB_FN(AsyncHostToDeviceTransferManager_TransferLiteral)
STUB_FN(Buffer_CopyRawToHostFuture)
STUB_FN(Device_PoisonExecution)
STUB_FN(Device_CreateAsyncTrackingEvent)
STUB_FN(AsyncTrackingEvent_Destroy)
STUB_FN(Executable_GetCompileOptions)
STUB_FN(Buffer_DonateWithControlDependency)

PJRT_Api make_api() {
  PJRT_Api api;
  std::memset(&api, 0, sizeof api);
  api.struct_size = PJRT_ABI_SIZE(PJRT_Api, PJRT_Event_Set);
  api.pjrt_api_version.struct_size = sizeof(PJRT_Api_Version);
  api.pjrt_api_version.major_version = PJRT_ABI_MAJOR;
  api.pjrt_api_version.minor_version = PJRT_ABI_MINOR;
#define SET(name) api.PJRT_##name = name
#define SET_STUB(name) api.PJRT_##name = Stub_##name
  SET(Error_Destroy);
  SET(Error_Message);
  SET(Error_GetCode);
  SET(Plugin_Initialize);
  SET(Plugin_Attributes);
  SET(Event_Destroy);
  SET(Event_IsReady);
  SET(Event_Error);
  SET(Event_Await);
  SET(Event_OnReady);
  SET(Client_Create);
  SET(Client_Destroy);
  SET(Client_PlatformName);
  SET(Client_ProcessIndex);
  SET(Client_PlatformVersion);
  SET(Client_Devices);
  SET(Client_AddressableDevices);
  SET(Client_LookupDevice);
  SET(Client_LookupAddressableDevice);
  SET(Client_AddressableMemories);
  SET(Client_Compile);
  SET(Client_DefaultDeviceAssignment);
  SET(Client_BufferFromHostBuffer);
  SET(DeviceDescription_Id);
  SET(DeviceDescription_ProcessIndex);
  SET(DeviceDescription_Attributes);
  SET(DeviceDescription_Kind);
  SET(DeviceDescription_DebugString);
  SET(DeviceDescription_ToString);
  SET(Device_GetDescription);
  SET(Device_IsAddressable);
  SET(Device_LocalHardwareId);
  SET(Device_AddressableMemories);
  SET(Device_DefaultMemory);
  SET(Device_MemoryStats);
  SET(Memory_Id);
  SET(Memory_Kind);
  SET(Memory_DebugString);
  SET(Memory_ToString);
  SET(Memory_AddressableByDevices);
  SET(Executable_Destroy);
  SET(Executable_Name);
  SET(Executable_NumReplicas);
  SET(Executable_NumPartitions);
  SET(Executable_NumOutputs);
  SET(Executable_SizeOfGeneratedCodeInBytes);
  SET(Executable_GetCostAnalysis);
  SET(Executable_OutputMemoryKinds);
  SET(Executable_OptimizedProgram);
  SET(Executable_Serialize);
  SET(LoadedExecutable_Destroy);
  SET(LoadedExecutable_GetExecutable);
  SET(LoadedExecutable_AddressableDevices);
  SET(LoadedExecutable_Delete);
  SET(LoadedExecutable_IsDeleted);
  SET(LoadedExecutable_Execute);
  SET(Executable_DeserializeAndLoad);
  SET(LoadedExecutable_Fingerprint);
  SET(Buffer_Destroy);
  SET(Buffer_ElementType);
  SET(Buffer_Dimensions);
  SET(Buffer_UnpaddedDimensions);
  SET(Buffer_DynamicDimensionIndices);
  SET(Buffer_GetMemoryLayout);
  SET(Buffer_OnDeviceSizeInBytes);
  SET(Buffer_Device);
  SET(Buffer_Memory);
  SET(Buffer_Delete);
  SET(Buffer_IsDeleted);
  SET(Buffer_CopyToDevice);
  SET(Buffer_ToHostBuffer);
  SET(Buffer_IsOnCpu);
  SET(Buffer_ReadyEvent);
  SET(Buffer_UnsafePointer);
  SET(Buffer_IncreaseExternalReferenceCount);
  SET(Buffer_DecreaseExternalReferenceCount);
  SET(Buffer_OpaqueDeviceMemoryDataPointer);
  SET_STUB(CopyToDeviceStream_Destroy);
  SET_STUB(CopyToDeviceStream_AddChunk);
  SET_STUB(CopyToDeviceStream_TotalBytes);
  SET_STUB(CopyToDeviceStream_GranuleSize);
  SET_STUB(CopyToDeviceStream_CurrentBytes);
  SET_STUB(TopologyDescription_Create);
  SET(TopologyDescription_Destroy);
  SET(TopologyDescription_PlatformName);
  SET(TopologyDescription_PlatformVersion);
  SET(TopologyDescription_GetDeviceDescriptions);
  SET_STUB(TopologyDescription_Serialize);
  SET(TopologyDescription_Attributes);
  SET_STUB(Compile);
  SET(Executable_OutputElementTypes);
  SET(Executable_OutputDimensions);
  SET(Buffer_CopyToMemory);
  SET(Client_CreateViewOfDeviceBuffer);
  SET(Executable_Fingerprint);
  SET(Client_TopologyDescription);
  SET(Executable_GetCompiledMemoryStats);
  SET(Memory_Kind_Id);
  SET(ExecuteContext_Create);
  SET(ExecuteContext_Destroy);
  SET(Buffer_CopyRawToHost);
  SET_STUB(AsyncHostToDeviceTransferManager_Destroy);
  SET_STUB(AsyncHostToDeviceTransferManager_TransferData);
  SET_STUB(Client_CreateBuffersForAsyncHostToDevice);
  SET_STUB(AsyncHostToDeviceTransferManager_RetrieveBuffer);
  SET_STUB(AsyncHostToDeviceTransferManager_Device);
  SET_STUB(AsyncHostToDeviceTransferManager_BufferCount);
  SET_STUB(AsyncHostToDeviceTransferManager_BufferSize);
  SET_STUB(AsyncHostToDeviceTransferManager_SetBufferError);
  SET_STUB(AsyncHostToDeviceTransferManager_AddMetadata);
  SET_STUB(Client_DmaMap);
  SET_STUB(Client_DmaUnmap);
  SET(Client_CreateUninitializedBuffer);
  SET_STUB(Client_UpdateGlobalProcessInfo);
  SET_STUB(TopologyDescription_Deserialize);
  SET_STUB(Client_CreateAliasBuffer);
  SET_STUB(Client_FulfillAliasBuffer);
  SET(LoadedExecutable_GetDeviceAssignment);
  SET_STUB(Client_CreateErrorBuffer);
  SET_STUB(AsyncHostToDeviceTransferManager_TransferLiteral);
  SET_STUB(Buffer_CopyRawToHostFuture);
  SET_STUB(Device_PoisonExecution);
  SET_STUB(Device_CreateAsyncTrackingEvent);
  SET_STUB(AsyncTrackingEvent_Destroy);
  SET_STUB(Executable_GetCompileOptions);
  SET_STUB(Buffer_DonateWithControlDependency);
  SET(Event_Create);
  SET(Event_Set);
#undef SET
#undef SET_STUB
  return api;
}

char* dup_cstr(const std::string& s) {
  char* p = static_cast<char*>(std::malloc(s.size() + 1));
  if (p) std::memcpy(p, s.c_str(), s.size() + 1);
  return p;
}

}  // namespace

extern "C" {

MFXP_EXPORT const PJRT_Api* GetPjrtApi(void) {
  static const PJRT_Api api = make_api();
  return &api;
}

MFXP_EXPORT int mfx_pjrt_inspect(const char* text, size_t size, char** json_out) {
  if (!json_out) return PJRT_Error_Code_INVALID_ARGUMENT;
  try {
    std::string src, route, err;
    if (!program_text(text ? text : "", text ? size : 0, src, route, err)) throw std::runtime_error(err);
    Compiled c = compile_text(src);
    *json_out = dup_cstr("{\"source\": \"" + route + "\", \"graph\": " + to_json(*c.main, &c.stats) +
                         ", \"plan\": " + c.plan->summary_json() + "}");
    return 0;
  } catch (const std::exception& e) {
    std::string m = e.what();
    std::string esc;
    for (char ch : m) {
      if (ch == '"' || ch == '\\') esc += '\\';
      if (ch == '\n') {
        esc += "\\n";
        continue;
      }
      esc += ch;
    }
    *json_out = dup_cstr("{\"error\": \"" + esc + "\"}");
    return PJRT_Error_Code_INVALID_ARGUMENT;
  }
}

MFXP_EXPORT void mfx_pjrt_free(char* p) { std::free(p); }

}  // extern "C"

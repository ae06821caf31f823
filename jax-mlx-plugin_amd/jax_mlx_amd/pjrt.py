"""ctypes driver of libpjrt_mi355x.so through the PJRT C API (GetPjrtApi).

This is what jaxlib's PJRT C-API client does for a plugin -- Client_Create,
Compile, BufferFromHostBuffer / CreateViewOfDeviceBuffer, Execute,
ToHostBuffer, Destroy -- made available in processes without jax (tests, the
benchmark).  Argument structs mirror include/pjrt_abi.h field for field.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_bool, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
PLUGIN_LIB = LIB_DIR / "libpjrt_mi355x.so"

# PJRT_Api function slots, in table order (PJRT C API 0.90).
SLOTS = """Error_Destroy Error_Message Error_GetCode Plugin_Initialize Plugin_Attributes Event_Destroy
Event_IsReady Event_Error Event_Await Event_OnReady Client_Create Client_Destroy Client_PlatformName
Client_ProcessIndex Client_PlatformVersion Client_Devices Client_AddressableDevices Client_LookupDevice
Client_LookupAddressableDevice Client_AddressableMemories Client_Compile Client_DefaultDeviceAssignment
Client_BufferFromHostBuffer DeviceDescription_Id DeviceDescription_ProcessIndex DeviceDescription_Attributes
DeviceDescription_Kind DeviceDescription_DebugString DeviceDescription_ToString Device_GetDescription
Device_IsAddressable Device_LocalHardwareId Device_AddressableMemories Device_DefaultMemory Device_MemoryStats
Memory_Id Memory_Kind Memory_DebugString Memory_ToString Memory_AddressableByDevices Executable_Destroy
Executable_Name Executable_NumReplicas Executable_NumPartitions Executable_NumOutputs
Executable_SizeOfGeneratedCodeInBytes Executable_GetCostAnalysis Executable_OutputMemoryKinds
Executable_OptimizedProgram Executable_Serialize LoadedExecutable_Destroy LoadedExecutable_GetExecutable
LoadedExecutable_AddressableDevices LoadedExecutable_Delete LoadedExecutable_IsDeleted LoadedExecutable_Execute
Executable_DeserializeAndLoad LoadedExecutable_Fingerprint Buffer_Destroy Buffer_ElementType Buffer_Dimensions
Buffer_UnpaddedDimensions Buffer_DynamicDimensionIndices Buffer_GetMemoryLayout Buffer_OnDeviceSizeInBytes
Buffer_Device Buffer_Memory Buffer_Delete Buffer_IsDeleted Buffer_CopyToDevice Buffer_ToHostBuffer Buffer_IsOnCpu
Buffer_ReadyEvent Buffer_UnsafePointer Buffer_IncreaseExternalReferenceCount Buffer_DecreaseExternalReferenceCount
Buffer_OpaqueDeviceMemoryDataPointer CopyToDeviceStream_Destroy CopyToDeviceStream_AddChunk
CopyToDeviceStream_TotalBytes CopyToDeviceStream_GranuleSize CopyToDeviceStream_CurrentBytes
TopologyDescription_Create TopologyDescription_Destroy TopologyDescription_PlatformName
TopologyDescription_PlatformVersion TopologyDescription_GetDeviceDescriptions TopologyDescription_Serialize
TopologyDescription_Attributes Compile Executable_OutputElementTypes Executable_OutputDimensions
Buffer_CopyToMemory Client_CreateViewOfDeviceBuffer Executable_Fingerprint Client_TopologyDescription
Executable_GetCompiledMemoryStats Memory_Kind_Id ExecuteContext_Create ExecuteContext_Destroy
Buffer_CopyRawToHost AsyncHostToDeviceTransferManager_Destroy AsyncHostToDeviceTransferManager_TransferData
Client_CreateBuffersForAsyncHostToDevice AsyncHostToDeviceTransferManager_RetrieveBuffer
AsyncHostToDeviceTransferManager_Device AsyncHostToDeviceTransferManager_BufferCount
AsyncHostToDeviceTransferManager_BufferSize AsyncHostToDeviceTransferManager_SetBufferError
AsyncHostToDeviceTransferManager_AddMetadata Client_DmaMap Client_DmaUnmap Client_CreateUninitializedBuffer
Client_UpdateGlobalProcessInfo TopologyDescription_Deserialize Client_CreateAliasBuffer Client_FulfillAliasBuffer
LoadedExecutable_GetDeviceAssignment Client_CreateErrorBuffer AsyncHostToDeviceTransferManager_TransferLiteral
Buffer_CopyRawToHostFuture Device_PoisonExecution Device_CreateAsyncTrackingEvent AsyncTrackingEvent_Destroy
Executable_GetCompileOptions Buffer_DonateWithControlDependency Event_Create Event_Set""".split()

# PJRT_Buffer_Type codes
PRED, S8, S16, S32, S64, U8, U16, U32, U64, F16, F32, F64, BF16 = 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13
ERROR_CODES = {0: "OK", 1: "CANCELLED", 2: "UNKNOWN", 3: "INVALID_ARGUMENT", 4: "DEADLINE_EXCEEDED",
               5: "NOT_FOUND", 6: "ALREADY_EXISTS", 7: "PERMISSION_DENIED", 8: "RESOURCE_EXHAUSTED",
               9: "FAILED_PRECONDITION", 10: "ABORTED", 11: "OUT_OF_RANGE", 12: "UNIMPLEMENTED",
               13: "INTERNAL", 14: "UNAVAILABLE", 15: "DATA_LOSS", 16: "UNAUTHENTICATED"}


class PjrtError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"PJRT {ERROR_CODES.get(code, code)}: {message}")
        self.code = code
        self.code_name = ERROR_CODES.get(code, str(code))
        self.message = message


def _args(name, fields):
    return type(name, (Structure,), {"_fields_": [("struct_size", c_size_t), ("extension_start", c_void_p)]
                                     + fields})


ErrorDestroyArgs = _args("ErrorDestroyArgs", [("error", c_void_p)])
ErrorMessageArgs = _args("ErrorMessageArgs", [("error", c_void_p), ("message", c_void_p), ("message_size", c_size_t)])
ErrorGetCodeArgs = _args("ErrorGetCodeArgs", [("error", c_void_p), ("code", c_int)])
PluginInitializeArgs = _args("PluginInitializeArgs", [])
ClientCreateArgs = _args("ClientCreateArgs", [
    ("create_options", c_void_p), ("num_options", c_size_t), ("kv_get_callback", c_void_p),
    ("kv_get_user_arg", c_void_p), ("kv_put_callback", c_void_p), ("kv_put_user_arg", c_void_p),
    ("client", c_void_p), ("kv_try_get_callback", c_void_p), ("kv_try_get_user_arg", c_void_p)])
ClientDestroyArgs = _args("ClientDestroyArgs", [("client", c_void_p)])
ClientPlatformNameArgs = _args("ClientPlatformNameArgs", [("client", c_void_p), ("platform_name", c_void_p),
                                                          ("platform_name_size", c_size_t)])
ClientDevicesArgs = _args("ClientDevicesArgs", [("client", c_void_p), ("devices", POINTER(c_void_p)),
                                                ("num_devices", c_size_t)])
Program = _args("Program", [("code", c_void_p), ("code_size", c_size_t), ("format", c_char_p),
                            ("format_size", c_size_t)])
ClientCompileArgs = _args("ClientCompileArgs", [("client", c_void_p), ("program", POINTER(Program)),
                                                ("compile_options", c_char_p), ("compile_options_size", c_size_t),
                                                ("executable", c_void_p)])
BufferFromHostArgs = _args("BufferFromHostArgs", [
    ("client", c_void_p), ("data", c_void_p), ("type", c_int), ("dims", POINTER(c_int64)), ("num_dims", c_size_t),
    ("byte_strides", POINTER(c_int64)), ("num_byte_strides", c_size_t), ("host_buffer_semantics", c_int),
    ("device", c_void_p), ("memory", c_void_p), ("device_layout", c_void_p), ("done_with_host_buffer", c_void_p),
    ("buffer", c_void_p)])
CreateViewArgs = _args("CreateViewArgs", [
    ("client", c_void_p), ("device_buffer_ptr", c_void_p), ("dims", POINTER(c_int64)), ("num_dims", c_size_t),
    ("element_type", c_int), ("layout", c_void_p), ("device", c_void_p), ("on_delete_callback", c_void_p),
    ("on_delete_callback_arg", c_void_p), ("stream", ctypes.c_ssize_t), ("buffer", c_void_p), ("memory", c_void_p)])
SerializeArgs = _args("SerializeArgs", [("executable", c_void_p), ("serialized_bytes", c_void_p),
                                        ("serialized_bytes_size", c_size_t), ("serialized_executable", c_void_p),
                                        ("serialized_executable_deleter", ctypes.CFUNCTYPE(None, c_void_p))])
DeserializeArgs = _args("DeserializeArgs", [("client", c_void_p), ("serialized_executable", c_void_p),
                                            ("serialized_executable_size", c_size_t),
                                            ("loaded_executable", c_void_p),
                                            ("overridden_serialized_compile_options", c_char_p),
                                            ("overridden_serialized_compile_options_size", c_size_t)])
ExecuteOptions = _args("ExecuteOptions", [
    ("send_callbacks", c_void_p), ("recv_callbacks", c_void_p), ("num_send_ops", c_size_t),
    ("num_recv_ops", c_size_t), ("launch_id", c_int), ("non_donatable_input_indices", c_void_p),
    ("num_non_donatable_input_indices", c_size_t), ("context", c_void_p), ("call_location", c_char_p),
    ("num_tasks", c_size_t), ("task_ids", c_void_p), ("incarnation_ids", c_void_p)])
ExecuteArgs = _args("ExecuteArgs", [
    ("executable", c_void_p), ("options", POINTER(ExecuteOptions)), ("argument_lists", POINTER(POINTER(c_void_p))),
    ("num_devices", c_size_t), ("num_args", c_size_t), ("output_lists", POINTER(POINTER(c_void_p))),
    ("device_complete_events", POINTER(c_void_p)), ("execute_device", c_void_p)])
ToHostArgs = _args("ToHostArgs", [("src", c_void_p), ("host_layout", c_void_p), ("dst", c_void_p),
                                  ("dst_size", c_size_t), ("event", c_void_p)])
BufferArgs = _args("BufferArgs", [("buffer", c_void_p)])
BufferDimsArgs = _args("BufferDimsArgs", [("buffer", c_void_p), ("dims", POINTER(c_int64)), ("num_dims", c_size_t)])
BufferTypeArgs = _args("BufferTypeArgs", [("buffer", c_void_p), ("type", c_int)])
BufferBoolArgs = _args("BufferBoolArgs", [("buffer", c_void_p), ("value", c_bool)])
BufferPtrArgs = _args("BufferPtrArgs", [("buffer", c_void_p), ("buffer_pointer", ctypes.c_uint64)])
EventArgs = _args("EventArgs", [("event", c_void_p)])
BufferEventArgs = _args("BufferEventArgs", [("buffer", c_void_p), ("event", c_void_p)])
GetExecutableArgs = _args("GetExecutableArgs", [("loaded_executable", c_void_p), ("executable", c_void_p)])
LoadedExecArgs = _args("LoadedExecArgs", [("executable", c_void_p)])
ExecNumOutputsArgs = _args("ExecNumOutputsArgs", [("executable", c_void_p), ("num_outputs", c_size_t)])
ExecOutTypesArgs = _args("ExecOutTypesArgs", [("executable", c_void_p), ("output_types", POINTER(c_int)),
                                              ("num_output_types", c_size_t)])
ExecOutDimsArgs = _args("ExecOutDimsArgs", [("executable", c_void_p), ("num_outputs", c_size_t),
                                            ("dims", POINTER(c_int64)), ("dim_sizes", POINTER(c_size_t))])
ExecNameArgs = _args("ExecNameArgs", [("executable", c_void_p), ("name", c_void_p), ("name_size", c_size_t)])


class NamedValue(Structure):
    class _V(ctypes.Union):
        _fields_ = [("string_value", c_void_p), ("int64_value", c_int64), ("int64_array_value", POINTER(c_int64)),
                    ("float_value", c_float), ("bool_value", c_bool)]

    _anonymous_ = ("v",)
    _fields_ = [("struct_size", c_size_t), ("extension_start", c_void_p), ("name", c_void_p), ("name_size", c_size_t),
                ("type", c_int), ("v", _V), ("value_size", c_size_t)]


CostArgs = _args("CostArgs", [("executable", c_void_p), ("num_properties", c_size_t),
                              ("properties", POINTER(NamedValue))])
PluginAttributesArgs = _args("PluginAttributesArgs", [("attributes", POINTER(NamedValue)),
                                                      ("num_attributes", c_size_t)])


def new(struct_type, **kw):
    a = struct_type(**kw)
    a.struct_size = ctypes.sizeof(struct_type)
    return a


class Api:
    """The function table of GetPjrtApi()."""

    _HEADER = 40  # struct_size, extension_start, PJRT_Api_Version (24 bytes)

    def __init__(self, path: str | Path | None = None):
        # MFX_PJRT_LIB selects another build of the plugin (the tests' sanitizer build).
        p = Path(path) if path else Path(os.environ.get("MFX_PJRT_LIB", PLUGIN_LIB))
        if not p.exists():
            raise FileNotFoundError(f"{p} is not built; run jax-mlx-plugin_amd/build.py")
        self.lib = ctypes.CDLL(str(p))
        self.lib.GetPjrtApi.restype = c_void_p
        self.base = self.lib.GetPjrtApi()
        self.struct_size = c_size_t.from_address(self.base).value
        self.version = (c_int.from_address(self.base + 32).value, c_int.from_address(self.base + 36).value)
        self.slots = {name: c_void_p.from_address(self.base + self._HEADER + 8 * i).value
                      for i, name in enumerate(SLOTS)}
        self._fn = {}
        self.lib.mfx_pjrt_inspect.argtypes = [c_char_p, c_size_t, POINTER(c_void_p)]
        self.lib.mfx_pjrt_free.argtypes = [c_void_p]

    def _f(self, name, restype=c_void_p):
        key = (name, restype)
        if key not in self._fn:
            self._fn[key] = ctypes.CFUNCTYPE(restype, c_void_p)(self.slots[name])
        return self._fn[key]

    def error_info(self, err: int):
        m = new(ErrorMessageArgs, error=err)
        self._f("Error_Message", None)(ctypes.addressof(m))
        msg = ctypes.string_at(m.message, m.message_size).decode() if m.message else ""
        g = new(ErrorGetCodeArgs, error=err)
        self._f("Error_GetCode")(ctypes.addressof(g))
        self._f("Error_Destroy", None)(ctypes.addressof(new(ErrorDestroyArgs, error=err)))
        return g.code, msg

    def call(self, name: str, args) -> None:
        err = self._f(name)(ctypes.addressof(args))
        if err:
            code, msg = self.error_info(err)
            raise PjrtError(code, msg)

    def inspect(self, text) -> dict:
        """Parse + rewrite + plan without a device (mfx_pjrt_inspect).  `text`
        is MLIR text (str) or program bytes (MLIR text, or bytecode that the
        process's MLIR runtime converts, as Client_Compile does)."""
        import json

        out = c_void_p()
        b = text.encode() if isinstance(text, str) else bytes(text)
        rc = self.lib.mfx_pjrt_inspect(b, len(b), ctypes.byref(out))
        s = ctypes.string_at(out.value).decode()
        self.lib.mfx_pjrt_free(out)
        doc = json.loads(s)
        if rc:
            raise PjrtError(rc, doc.get("error", ""))
        return doc


_TORCH_TO_PJRT = None


def _torch_types():
    global _TORCH_TO_PJRT
    if _TORCH_TO_PJRT is None:
        import torch

        _TORCH_TO_PJRT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int32: S32,
                          torch.int64: S64, torch.bool: PRED, torch.uint8: U8, torch.float64: F64}
    return _TORCH_TO_PJRT


class Buffer:
    def __init__(self, client: "Client", handle: int, keepalive=None):
        self.client = client
        self.handle = handle
        self._keep = keepalive

    @property
    def dims(self):
        a = new(BufferDimsArgs, buffer=self.handle)
        self.client.api.call("Buffer_Dimensions", a)
        return tuple(a.dims[i] for i in range(a.num_dims))

    @property
    def type(self):
        a = new(BufferTypeArgs, buffer=self.handle)
        self.client.api.call("Buffer_ElementType", a)
        return a.type

    def device_pointer(self) -> int:
        a = new(BufferPtrArgs, buffer=self.handle)
        self.client.api.call("Buffer_UnsafePointer", a)
        return a.buffer_pointer

    def await_ready(self):
        ev = new(BufferEventArgs, buffer=self.handle)
        self.client.api.call("Buffer_ReadyEvent", ev)
        self.client.api.call("Event_Await", new(EventArgs, event=ev.event))
        self.client.api.call("Event_Destroy", new(EventArgs, event=ev.event))

    def to_torch(self):
        """Copies to a new host torch tensor (Buffer_ToHostBuffer)."""
        import torch

        inv = {v: k for k, v in _torch_types().items()}
        t = torch.empty(self.dims, dtype=inv[self.type])
        q = new(ToHostArgs, src=self.handle)
        self.client.api.call("Buffer_ToHostBuffer", q)  # size query
        if q.dst_size != t.numel() * t.element_size():
            raise PjrtError(13, f"ToHostBuffer size {q.dst_size} != {t.numel() * t.element_size()}")
        a = new(ToHostArgs, src=self.handle, dst=t.data_ptr(), dst_size=q.dst_size)
        self.client.api.call("Buffer_ToHostBuffer", a)
        if a.event:
            self.client.api.call("Event_Await", new(EventArgs, event=a.event))
            self.client.api.call("Event_Destroy", new(EventArgs, event=a.event))
        return t

    def destroy(self):
        if self.handle:
            self.client.api.call("Buffer_Destroy", new(BufferArgs, buffer=self.handle))
            self.handle = 0
            self._keep = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Executable:
    def __init__(self, client: "Client", handle: int):
        self.client = client
        self.handle = handle
        g = new(GetExecutableArgs, loaded_executable=handle)
        client.api.call("LoadedExecutable_GetExecutable", g)
        self.exe = g.executable

    @property
    def num_outputs(self) -> int:
        a = new(ExecNumOutputsArgs, executable=self.exe)
        self.client.api.call("Executable_NumOutputs", a)
        return a.num_outputs

    @property
    def output_types(self):
        a = new(ExecOutTypesArgs, executable=self.exe)
        self.client.api.call("Executable_OutputElementTypes", a)
        return [a.output_types[i] for i in range(a.num_output_types)]

    @property
    def output_dims(self):
        a = new(ExecOutDimsArgs, executable=self.exe)
        self.client.api.call("Executable_OutputDimensions", a)
        out, k = [], 0
        for i in range(a.num_outputs):
            n = a.dim_sizes[i]
            out.append(tuple(a.dims[k + j] for j in range(n)))
            k += n
        return out

    @property
    def name(self) -> str:
        a = new(ExecNameArgs, executable=self.exe)
        self.client.api.call("Executable_Name", a)
        return ctypes.string_at(a.name, a.name_size).decode()

    def cost_analysis(self) -> dict:
        a = new(CostArgs, executable=self.exe)
        self.client.api.call("Executable_GetCostAnalysis", a)
        out = {}
        for i in range(a.num_properties):
            nv = a.properties[i]
            out[ctypes.string_at(nv.name, nv.name_size).decode()] = nv.float_value
        return out

    def execute(self, args, wait: bool = True):
        """Runs the executable on `args` (Buffers); returns output Buffers."""
        n_out = self.num_outputs
        arg_arr = (c_void_p * max(1, len(args)))(*[b.handle for b in args])
        arg_lists = (POINTER(c_void_p) * 1)(ctypes.cast(arg_arr, POINTER(c_void_p)))
        out_arr = (c_void_p * max(1, n_out))()
        out_lists = (POINTER(c_void_p) * 1)(ctypes.cast(out_arr, POINTER(c_void_p)))
        events = (c_void_p * 1)()
        opts = new(ExecuteOptions)
        a = new(ExecuteArgs, executable=self.handle, options=ctypes.pointer(opts), argument_lists=arg_lists,
                num_devices=1, num_args=len(args), output_lists=out_lists,
                device_complete_events=ctypes.cast(events, POINTER(c_void_p)))
        self.client.api.call("LoadedExecutable_Execute", a)
        if events[0]:
            if wait:
                self.client.api.call("Event_Await", new(EventArgs, event=events[0]))
            self.client.api.call("Event_Destroy", new(EventArgs, event=events[0]))
        return [Buffer(self.client, out_arr[i]) for i in range(n_out)]

    def serialize(self) -> bytes:
        """Executable_Serialize: the plugin's serialized form (its bytes are
        copied out and the plugin's copy freed with its deleter)."""
        a = new(SerializeArgs, executable=self.exe)
        self.client.api.call("Executable_Serialize", a)
        data = ctypes.string_at(a.serialized_bytes, a.serialized_bytes_size)
        a.serialized_executable_deleter(a.serialized_executable)
        return data

    def destroy(self):
        if self.handle:
            self.client.api.call("Executable_Destroy", new(LoadedExecArgs, executable=self.exe))
            self.client.api.call("LoadedExecutable_Destroy", new(LoadedExecArgs, executable=self.handle))
            self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Client:
    """A PJRT client of the plugin (one per process is enough)."""

    def __init__(self, api: Api | None = None):
        self.api = api or Api()
        self.api.call("Plugin_Initialize", new(PluginInitializeArgs))
        a = new(ClientCreateArgs)
        self.api.call("Client_Create", a)
        self.handle = a.client

    @property
    def platform_name(self) -> str:
        a = new(ClientPlatformNameArgs, client=self.handle)
        self.api.call("Client_PlatformName", a)
        return ctypes.string_at(a.platform_name, a.platform_name_size).decode()

    def devices(self):
        a = new(ClientDevicesArgs, client=self.handle)
        self.api.call("Client_Devices", a)
        return [a.devices[i] for i in range(a.num_devices)]

    def compile(self, mlir_text: str) -> Executable:
        code = mlir_text.encode()
        buf = ctypes.create_string_buffer(code, len(code))
        prog = new(Program, code=ctypes.cast(buf, c_void_p), code_size=len(code), format=b"mlir", format_size=4)
        a = new(ClientCompileArgs, client=self.handle, program=ctypes.pointer(prog), compile_options=b"",
                compile_options_size=0)
        self.api.call("Client_Compile", a)
        return Executable(self, a.executable)

    def deserialize(self, blob: bytes) -> Executable:
        """Executable_DeserializeAndLoad of Executable.serialize()'s bytes."""
        buf = ctypes.create_string_buffer(blob, len(blob))
        a = new(DeserializeArgs, client=self.handle, serialized_executable=ctypes.cast(buf, c_void_p),
                serialized_executable_size=len(blob))
        self.api.call("Executable_DeserializeAndLoad", a)
        return Executable(self, a.loaded_executable)

    def buffer_from_host(self, tensor, byte_strides=None) -> Buffer:
        """BufferFromHostBuffer from a host torch tensor (or numpy array)."""
        import torch

        t = tensor if isinstance(tensor, torch.Tensor) else torch.from_numpy(tensor)
        if t.is_cuda:
            raise ValueError("buffer_from_host takes a host tensor; use buffer_view for device tensors")
        if byte_strides is None:
            t = t.contiguous()
        dims = (c_int64 * max(1, t.dim()))(*t.shape)
        bs = None
        if byte_strides is not None:
            bs = (c_int64 * len(byte_strides))(*byte_strides)
        a = new(BufferFromHostArgs, client=self.handle, data=t.data_ptr(), type=_torch_types()[t.dtype], dims=dims,
                num_dims=t.dim(), byte_strides=bs, num_byte_strides=len(byte_strides) if byte_strides else 0,
                host_buffer_semantics=0)
        self.api.call("Client_BufferFromHostBuffer", a)
        if a.done_with_host_buffer:
            self.api.call("Event_Destroy", new(EventArgs, event=a.done_with_host_buffer))
        return Buffer(self, a.buffer)

    def buffer_view(self, tensor) -> Buffer:
        """Zero-copy PJRT buffer over a contiguous device torch tensor
        (Client_CreateViewOfDeviceBuffer); the tensor is kept alive."""
        if not tensor.is_cuda or not tensor.is_contiguous():
            raise ValueError("buffer_view needs a contiguous device tensor")
        dims = (c_int64 * max(1, tensor.dim()))(*tensor.shape)
        a = new(CreateViewArgs, client=self.handle, device_buffer_ptr=tensor.data_ptr(), dims=dims,
                num_dims=tensor.dim(), element_type=_torch_types()[tensor.dtype])
        self.api.call("Client_CreateViewOfDeviceBuffer", a)
        return Buffer(self, a.buffer, keepalive=tensor)

    def destroy(self):
        if self.handle:
            self.api.call("Client_Destroy", new(ClientDestroyArgs, client=self.handle))
            self.handle = 0


def smoke_check(oracle) -> None:
    """Compiles a LayerNorm module through Client_Compile, runs it with
    Execute and checks it against the oracle (used by __graft_entry__.smoke)."""
    import sys

    import numpy as np
    import torch

    tests_dir = Path(__file__).resolve().parents[2] / "tests"
    if str(tests_dir) not in sys.path:
        sys.path.insert(0, str(tests_dir))
    import mlir_modules

    client = Client()
    exe = client.compile(mlir_modules.layer_norm_module(shape=(4, 512)))
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    bufs = [client.buffer_from_host(a) for a in (x, g, b)]
    out = exe.execute(bufs)[0].to_torch().numpy().astype(np.float64)
    err = np.abs(out - oracle.layer_norm(x, g, b, 1e-5)).max()
    print(f"PJRT Compile/Execute layer_norm [4,512] on {client.platform_name}: max abs err {err:.2e}")
    assert err <= 1e-5, err
    for buf in bufs:
        buf.destroy()
    exe.destroy()
    client.destroy()
    del torch

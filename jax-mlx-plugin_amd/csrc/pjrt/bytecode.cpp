// Program bytes -> MLIR text.
//
// jaxlib hands PJRT plugins the module as a serialized StableHLO portable
// artifact ("ML\xefR" bytecode); other hosts (Reactant.jl, C drivers) may hand
// MLIR text.  The plugin's parser reads text, so bytecode is turned into text
// first, by whichever MLIR runtime the calling process already holds.  Two
// routes are tried in the reference's order (src/jax_mlx_pjrt.cpp:671-830):
//
//   1. the MLIR C API exported into the process (Reactant.jl and other hosts
//      without Python): stablehloDeserializePortableArtifactNoError, with
//      mlirModuleCreateParse as the fallback, printed by mlirOperationPrint
//      (reference :674-745);
//   2. the jaxlib of a running Python interpreter, through
//      jax_mlx_amd._bytecode.to_text() (reference :749-822).
//
// Every symbol is resolved with dlsym at run time, so the library loads in any
// process; with neither runtime present, only MLIR text is accepted.
#include <dlfcn.h>

#include <cstring>
#include <string>

namespace mfxp {

bool is_mlir_bytecode(const char* data, size_t size) {
  return size >= 4 && data[0] == 'M' && data[1] == 'L' && (unsigned char)data[2] == 0xEF && data[3] == 'R';
}

namespace {

// ---- route 1: the MLIR C API ----------------------------------------------
//
// The C API passes its handles as one-pointer structs and strings as
// (data, length) pairs, by value; these mirror that layout.
struct MHandle {
  void* ptr;
};
struct MString {
  const char* data;
  size_t length;
};

struct MlirCApi {
  MHandle (*context_create)();
  void (*context_destroy)(MHandle);
  void (*allow_unregistered)(MHandle, bool);
  void (*load_all_dialects)(MHandle);
  MHandle (*deserialize_artifact)(MString, MHandle);
  MHandle (*module_parse)(MHandle, MString);
  void (*module_destroy)(MHandle);
  MHandle (*module_operation)(MHandle);
  void (*operation_print)(MHandle, void (*)(MString, void*), void*);
  // A usable route needs a context, a module source and a printer.
  bool usable() const {
    return context_create && module_operation && operation_print && (deserialize_artifact || module_parse);
  }
};

template <class F>
void bind(F& f, const char* name) {
  f = reinterpret_cast<F>(dlsym(RTLD_DEFAULT, name));
}

// Resolved per call: a host may load its MLIR runtime after this library.
MlirCApi find_mlir_capi() {
  MlirCApi a{};
  bind(a.context_create, "mlirContextCreate");
  bind(a.context_destroy, "mlirContextDestroy");
  bind(a.allow_unregistered, "mlirContextSetAllowUnregisteredDialects");
  bind(a.load_all_dialects, "mlirContextLoadAllAvailableDialects");
  bind(a.deserialize_artifact, "stablehloDeserializePortableArtifactNoError");
  bind(a.module_parse, "mlirModuleCreateParse");
  bind(a.module_destroy, "mlirModuleDestroy");
  bind(a.module_operation, "mlirModuleGetOperation");
  bind(a.operation_print, "mlirOperationPrint");
  return a;
}

void append_chunk(MString s, void* user) { static_cast<std::string*>(user)->append(s.data, s.length); }

// Returns true with the module's text; false with the reason otherwise.
bool via_mlir_capi(const MlirCApi& api, const char* data, size_t size, std::string& text, std::string& err) {
  MHandle ctx = api.context_create();
  if (!ctx.ptr) {
    err = "mlirContextCreate returned no context";
    return false;
  }
  if (api.allow_unregistered) api.allow_unregistered(ctx, true);
  if (api.load_all_dialects) api.load_all_dialects(ctx);
  const MString in{data, size};
  MHandle mod{nullptr};
  if (api.deserialize_artifact) mod = api.deserialize_artifact(in, ctx);
  if (!mod.ptr && api.module_parse) mod = api.module_parse(ctx, in);
  bool ok = false;
  if (mod.ptr) {
    text.clear();
    api.operation_print(api.module_operation(mod), append_chunk, &text);
    ok = !text.empty();
    if (!ok) err = "mlirOperationPrint produced no text";
    if (api.module_destroy) api.module_destroy(mod);
  } else {
    err = "the MLIR C API could neither deserialize nor parse the module";
  }
  if (api.context_destroy) api.context_destroy(ctx);
  return ok;
}

// ---- route 2: the calling process's Python and jaxlib ------------------------

typedef void PyObject;
struct PyApi {
  int (*Py_IsInitialized)();
  int (*PyGILState_Ensure)();
  void (*PyGILState_Release)(int);
  PyObject* (*PyImport_ImportModule)(const char*);
  PyObject* (*PyObject_GetAttrString)(PyObject*, const char*);
  PyObject* (*PyBytes_FromStringAndSize)(const char*, long);
  PyObject* (*PyObject_CallFunctionObjArgs)(PyObject*, ...);
  const char* (*PyUnicode_AsUTF8AndSize)(PyObject*, long*);
  void (*Py_DecRef)(PyObject*);
  void (*PyErr_Fetch)(PyObject**, PyObject**, PyObject**);
  PyObject* (*PyObject_Str)(PyObject*);
  bool ok = false;
};

PyApi load_py_api() {
  PyApi a{};
#define SYM(name)          \
  bind(a.name, #name);     \
  if (!a.name) return a;
  SYM(Py_IsInitialized)
  SYM(PyGILState_Ensure)
  SYM(PyGILState_Release)
  SYM(PyImport_ImportModule)
  SYM(PyObject_GetAttrString)
  SYM(PyBytes_FromStringAndSize)
  SYM(PyObject_CallFunctionObjArgs)
  SYM(PyUnicode_AsUTF8AndSize)
  SYM(Py_DecRef)
  SYM(PyErr_Fetch)
  SYM(PyObject_Str)
#undef SYM
  a.ok = true;
  return a;
}

std::string py_error(const PyApi& a) {
  PyObject *t = nullptr, *v = nullptr, *tb = nullptr;
  a.PyErr_Fetch(&t, &v, &tb);
  std::string msg = "Python error";
  if (v) {
    PyObject* s = a.PyObject_Str(v);
    if (s) {
      long n = 0;
      const char* c = a.PyUnicode_AsUTF8AndSize(s, &n);
      if (c) msg.assign(c, (size_t)n);
      a.Py_DecRef(s);
    }
  }
  if (t) a.Py_DecRef(t);
  if (v) a.Py_DecRef(v);
  if (tb) a.Py_DecRef(tb);
  return msg;
}

bool via_python(const PyApi& api, const char* data, size_t size, std::string& text, std::string& err) {
  const int gil = api.PyGILState_Ensure();
  bool ok = false;
  PyObject* mod = api.PyImport_ImportModule("jax_mlx_amd._bytecode");
  PyObject* fn = mod ? api.PyObject_GetAttrString(mod, "to_text") : nullptr;
  PyObject* bytes = fn ? api.PyBytes_FromStringAndSize(data, (long)size) : nullptr;
  PyObject* res = bytes ? api.PyObject_CallFunctionObjArgs(fn, bytes, nullptr) : nullptr;
  if (res) {
    long n = 0;
    const char* c = api.PyUnicode_AsUTF8AndSize(res, &n);
    if (c) {
      text.assign(c, (size_t)n);
      ok = true;
    }
  }
  if (!ok) err = "jax_mlx_amd._bytecode.to_text: " + py_error(api);
  for (PyObject* o : {res, bytes, fn, mod})
    if (o) api.Py_DecRef(o);
  api.PyGILState_Release(gil);
  return ok;
}

}  // namespace

// MLIR text of a program: the bytes themselves when they are not bytecode,
// otherwise the first route that converts them.  `route` names what was used
// ("text", "mlir-capi", "python").  On failure `err` says what each route
// reported, or that neither exists in this process.
bool program_text(const char* data, size_t size, std::string& text, std::string& route, std::string& err) {
  if (!is_mlir_bytecode(data, size)) {
    text.assign(data, size);
    route = "text";
    return true;
  }
  std::string why;
  const MlirCApi capi = find_mlir_capi();
  if (capi.usable()) {
    std::string e;
    if (via_mlir_capi(capi, data, size, text, e)) {
      route = "mlir-capi";
      return true;
    }
    why = "MLIR C API: " + e;
  }
  if (why.empty())
    why = "no MLIR C API (mlirContextCreate, stablehloDeserializePortableArtifactNoError, mlirOperationPrint)";
  static const PyApi py = load_py_api();
  if (py.ok && py.Py_IsInitialized()) {
    std::string e;
    if (via_python(py, data, size, text, e)) {
      route = "python";
      return true;
    }
    err = why + "; " + e;
  } else {
    err = why + "; no Python interpreter in this process; pass MLIR text instead";
  }
  return false;
}

}  // namespace mfxp

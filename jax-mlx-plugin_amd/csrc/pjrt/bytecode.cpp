// MLIR bytecode (StableHLO portable artifact) -> MLIR text.
//
// jaxlib hands PJRT plugins the module as a serialized portable artifact
// ("ML\xefR" bytecode).  Deserialising it needs MLIR's StableHLO dialect,
// which lives in the jaxlib already loaded in the calling process; like the
// reference (src/jax_mlx_pjrt.cpp:749-822) the plugin calls into that
// interpreter, here through jax_mlx_amd._bytecode.to_text().  The Python C-API
// symbols are resolved with dlsym at run time so the library also loads in
// processes without Python (the C++ / ctypes test drivers), where only MLIR
// text is accepted.
#include <dlfcn.h>

#include <cstring>
#include <string>

namespace mfxp {

bool is_mlir_bytecode(const char* data, size_t size) {
  return size >= 4 && data[0] == 'M' && data[1] == 'L' && (unsigned char)data[2] == 0xEF && data[3] == 'R';
}

namespace {

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

PyApi load_api() {
  PyApi a{};
  void* h = RTLD_DEFAULT;
#define SYM(name)                                                  \
  a.name = reinterpret_cast<decltype(a.name)>(dlsym(h, #name));   \
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

}  // namespace

bool bytecode_to_text(const char* data, size_t size, std::string& text, std::string& err) {
  static const PyApi api = load_api();
  if (!api.ok || !api.Py_IsInitialized()) {
    err = "bytecode needs the jaxlib of a running Python process; pass MLIR text instead";
    return false;
  }
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
  if (!ok) err = py_error(api);
  for (PyObject* o : {res, bytes, fn, mod})
    if (o) api.Py_DecRef(o);
  api.PyGILState_Release(gil);
  return ok;
}

}  // namespace mfxp

/* Test double of the MLIR C API symbols libpjrt_mi355x.so resolves with
 * dlsym to turn MLIR bytecode into text (csrc/pjrt/bytecode.cpp, route 1).
 * Not MLIR: a "portable artifact" here is the bytecode magic "ML\xefR"
 * followed by a tag and MLIR text.
 *   "ML\xefR" "VHLO:" <text>   stablehloDeserializePortableArtifactNoError succeeds
 *   "ML\xefR" "PARSE:" <text>  that fails, mlirModuleCreateParse succeeds
 *   anything else              both fail
 * mlirOperationPrint hands the text to the callback in 7-byte chunks.
 * mlir_stub_live() counts contexts and modules not yet destroyed;
 * mlir_stub_calls() counts dialect set-up calls. */
#include <stdbool.h>
#include <stdlib.h>
#include <string.h>

typedef struct { void* ptr; } Handle;
typedef struct { const char* data; size_t length; } Str;
typedef struct { char* text; size_t n; } StubModule;

static int live = 0, setup_calls = 0;

int mlir_stub_live(void) { return live; }
int mlir_stub_calls(void) { return setup_calls; }

Handle mlirContextCreate(void) { ++live; Handle h = {malloc(1)}; return h; }
void mlirContextDestroy(Handle c) { --live; free(c.ptr); }
void mlirContextSetAllowUnregisteredDialects(Handle c, bool allow) { (void)c; setup_calls += allow ? 1 : 0; }
void mlirContextLoadAllAvailableDialects(Handle c) { (void)c; ++setup_calls; }

static Handle module_after(Str in, const char* tag) {
  Handle h = {NULL};
  size_t t = strlen(tag);
  if (in.length < 4 + t || memcmp(in.data, "ML\xefR", 4) != 0 || memcmp(in.data + 4, tag, t) != 0) return h;
  StubModule* m = malloc(sizeof *m);
  m->n = in.length - 4 - t;
  m->text = malloc(m->n);
  memcpy(m->text, in.data + 4 + t, m->n);
  ++live;
  h.ptr = m;
  return h;
}

Handle stablehloDeserializePortableArtifactNoError(Str in, Handle ctx) { (void)ctx; return module_after(in, "VHLO:"); }
Handle mlirModuleCreateParse(Handle ctx, Str in) { (void)ctx; return module_after(in, "PARSE:"); }
void mlirModuleDestroy(Handle m) {
  StubModule* s = m.ptr;
  free(s->text);
  free(s);
  --live;
}
Handle mlirModuleGetOperation(Handle m) { return m; }
void mlirOperationPrint(Handle op, void (*cb)(Str, void*), void* user) {
  const StubModule* s = op.ptr;
  for (size_t i = 0; i < s->n; i += 7) {
    Str chunk = {s->text + i, s->n - i < 7 ? s->n - i : 7};
    cb(chunk, user);
  }
}

/* lokinfer MI355X runtime: compiled models behind a plain-C boundary.
 *
 * Replaces the reference's C++ runtime surface (lariaus/lokinfer include/lokinfer/runtime/runtime.h:84-124
 * Executable::create / run; include/lokinfer/ir/binary.h:22-43 readModelFile / writeModelFile; text.h printModel /
 * parseModel; compiler/passes.h runPasses / internalize) and its nanobind binding (python/ext/module.cpp:
 * compile_text, create_executable, load_model, save_model). Models use the reference's text IR and .lkm v2 format.
 *
 * Errors: functions return NULL or a nonzero status; lk_last_error() (include/lokinfer_hip.h) has the message.
 * Strings and byte buffers the library returns are released with lk_free.
 */
#ifndef LOKINFER_RT_H
#define LOKINFER_RT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lk_model lk_model;
typedef struct lk_exe lk_exe;

/* dtype codes: the .lkm encoding (f32 0, f16 1, bf16 2, i8 3, u8 4, i16 5, i32 6, i64 7, bool 8) */
typedef struct {
  void* data;        /* device pointer (a host pointer to an 8-byte slot for a scalar input) */
  int64_t shape[8];
  int32_t rank;
  int32_t dtype;
} lk_tensor;

void lk_free(void* p);

/* ---- models (reference: parseModel text.h:17-20, readModelFile / writeModelFile binary.h:22-27) ---- */
lk_model* lk_model_parse(const char* text);
lk_model* lk_model_load(const char* path);                         /* .lkm v1 / v2, mmapped, constants zero-copy */
lk_model* lk_model_from_bytes(const void* bytes, uint64_t size);   /* copies the bytes */
int lk_model_save(const lk_model* m, const char* path);
int lk_model_to_bytes(const lk_model* m, void** bytes, uint64_t* size);
char* lk_model_print(const lk_model* m);
int lk_model_verify(const lk_model* m);
/* passes: comma-separated names (dce, bufferize, plan-memory, hoist-init) or "pipeline"; verifies after each */
int lk_model_run_passes(lk_model* m, const char* passes);
/* the bytes of internal constant `name` (copy != 0: the model keeps its own copy; else `bytes` must outlive it) */
int lk_model_set_constant(lk_model* m, const char* name, const void* bytes, uint64_t size, int copy);
/* const.external -> const.internal for the n externals given (host bytes, copied) (reference internalize) */
int lk_model_internalize(lk_model* m, int n, const char* const* names, const void* const* bytes, const uint64_t* sizes);
int lk_model_num_inputs(const lk_model* m);
int lk_model_num_outputs(const lk_model* m);
/* 1 if exec input i is mutable (written in place), else 0 */
int lk_model_input_is_mutable(const lk_model* m, int i);
void lk_model_free(lk_model* m);
/* the canonical text of a dim expression ("2*(N + 1)" -> "2*N + 2"); NULL if it does not parse */
char* lk_dim_canonical(const char* text);

/* bake-init (reference: rt::bakeInit, runtime/bake_init.h:19-27): runs `m`'s init once with the externals bound
 * (as lk_exe_create) and returns a new model in which every init result that is computed data (a plain
 * buffer.alloc written by init kernels, or a view of one) is a const.internal holding that data, resident where the
 * kernel that wrote it runs; init ops nothing needs any more are removed. Arena, persistent and output buffers,
 * constants, and models whose init defines symbols (dim.read, mem.plan) are left alone. stats (may be NULL):
 * [baked, baked bytes, init ops before, init ops after]. NULL on error (lk_last_error). */
lk_model* lk_model_bake_init(const lk_model* m, int n_ext, const char* const* names, void* const* ptrs,
                             const uint64_t* sizes, const int* on_device, void* stream, uint64_t* stats);

/* ---- executables (reference: Executable::create / run, runtime.h:84-95) ----
 * create: the model must be in buffer form (after bufferize). Externals are bound by name: device pointers
 * (on_device != 0, borrowed: they must outlive the executable) or host bytes (uploaded once). Uploads every
 * constant into one device arena and runs init on `stream`. flags: bit 0 = capture statically shaped calls into
 * hipGraphs; bits 8-11 = the most HIP streams a statically shaped call may use (0 or 1: one stream). Kernels are
 * assigned to streams from their data dependencies. The executable keeps the model alive. */
lk_exe* lk_exe_create(lk_model* m, int n_ext, const char* const* names, void* const* ptrs, const uint64_t* sizes,
                      const int* on_device, void* stream, int flags);
/* run: enqueues one call on `stream`; outputs point into memory the executable owns, valid until its next call.
 * flags: bit 0 = synchronize and report device-side data errors. Calls of one executable must be stream-ordered. */
int lk_exe_run(lk_exe* e, int n_in, const lk_tensor* inputs, int max_out, lk_tensor* outputs, int* n_out,
               void* stream, int flags);
/* model arena bytes (incl. the re-placed temporaries), call arena bytes, captured graphs, streams in use */
int lk_exe_stats(const lk_exe* e, uint64_t* model_bytes, uint64_t* call_bytes, int* graphs, int* streams);
void lk_exe_free(lk_exe* e);

#ifdef __cplusplus
}
#endif

#endif /* LOKINFER_RT_H */

// C-ABI of the runtime (include/lokinfer_rt.h).
#include <cstdlib>
#include <cstring>

#include "executable.h"
#include "lokinfer_hip.h"
#include "lokinfer_rt.h"

struct lk_model {
  std::shared_ptr<lkrt::Model> m;
};

struct lk_exe {
  std::unique_ptr<lkrt::Executable> e;
};

namespace {

int fail(const lkrt::Status& s) {
  lkh::setLastError(s.message());
  return 1;
}

template <typename T>
T* failNull(const lkrt::Status& s) {
  lkh::setLastError(s.message());
  return nullptr;
}

lk_model* wrap(std::unique_ptr<lkrt::Model> m) {
  auto* w = new lk_model;
  w->m = std::move(m);
  return w;
}

char* dupString(const std::string& s) {
  char* p = static_cast<char*>(std::malloc(s.size() + 1));
  if (p) std::memcpy(p, s.c_str(), s.size() + 1);
  return p;
}

}  // namespace

extern "C" {

void lk_free(void* p) { std::free(p); }

lk_model* lk_model_parse(const char* text) {
  if (!text) return failNull<lk_model>(lkrt::Status::error("null text"));
  lkrt::Status st;
  auto m = lkrt::parseModel(text, st);
  if (!m) return failNull<lk_model>(st);
  if (lkrt::Status v = lkrt::verifyModel(*m); !v) return failNull<lk_model>(v);
  return wrap(std::move(m));
}

lk_model* lk_model_load(const char* path) {
  lkrt::Status st;
  auto m = lkrt::readLkmFile(path ? path : "", st);
  if (!m) return failNull<lk_model>(st);
  if (lkrt::Status v = lkrt::verifyModel(*m); !v) return failNull<lk_model>(v);
  return wrap(std::move(m));
}

lk_model* lk_model_from_bytes(const void* bytes, uint64_t size) {
  if (!bytes) return failNull<lk_model>(lkrt::Status::error("null bytes"));
  auto copy = std::make_shared<std::vector<uint8_t>>(static_cast<const uint8_t*>(bytes),
                                                     static_cast<const uint8_t*>(bytes) + size);
  lkrt::Status st;
  auto m = lkrt::readLkm(copy->data(), copy->size(), copy, st);
  if (!m) return failNull<lk_model>(st);
  if (lkrt::Status v = lkrt::verifyModel(*m); !v) return failNull<lk_model>(v);
  return wrap(std::move(m));
}

int lk_model_save(const lk_model* m, const char* path) {
  if (!m || !path) return fail(lkrt::Status::error("null model or path"));
  lkrt::Status s = lkrt::writeLkmFile(*m->m, path);
  return s ? 0 : fail(s);
}

int lk_model_to_bytes(const lk_model* m, void** bytes, uint64_t* size) {
  if (!m || !bytes || !size) return fail(lkrt::Status::error("null argument"));
  lkrt::Status st;
  std::vector<uint8_t> b = lkrt::writeLkm(*m->m, st);
  if (!st) return fail(st);
  *bytes = std::malloc(std::max<size_t>(b.size(), 1));
  if (!*bytes) return fail(lkrt::Status::error("out of memory"));
  std::memcpy(*bytes, b.data(), b.size());
  *size = b.size();
  return 0;
}

char* lk_model_print(const lk_model* m) { return m ? dupString(lkrt::printModel(*m->m)) : nullptr; }

int lk_model_verify(const lk_model* m) {
  if (!m) return fail(lkrt::Status::error("null model"));
  lkrt::Status s = lkrt::verifyModel(*m->m);
  return s ? 0 : fail(s);
}

int lk_model_run_passes(lk_model* m, const char* passes) {
  if (!m || !passes) return fail(lkrt::Status::error("null argument"));
  std::vector<std::string> names;
  const std::string list = passes;
  if (list == "pipeline") {
    names = lkrt::defaultPipeline();
  } else {
    size_t b = 0;
    while (b <= list.size()) {
      size_t e = list.find(',', b);
      if (e == std::string::npos) e = list.size();
      if (e > b) names.push_back(list.substr(b, e - b));
      b = e + 1;
    }
  }
  for (const std::string& n : names)
    if (lkrt::Status s = lkrt::runPass(*m->m, n); !s) return fail(s);
  return 0;
}

int lk_model_set_constant(lk_model* m, const char* name, const void* bytes, uint64_t size, int copy) {
  if (!m || !name) return fail(lkrt::Status::error("null argument"));
  lkrt::Constant* c = m->m->findConstant(name);
  if (!c) return fail(lkrt::Status::error(std::string("no internal constant '") + name + "'"));
  if (copy) {
    auto owned = std::make_shared<std::vector<uint8_t>>(static_cast<const uint8_t*>(bytes),
                                                        static_cast<const uint8_t*>(bytes) + size);
    c->bytes = owned->data();
    c->owner = owned;
  } else {
    c->bytes = static_cast<const uint8_t*>(bytes);
    c->owner = nullptr;
  }
  c->size = size;
  return 0;
}

int lk_model_internalize(lk_model* m, int n, const char* const* names, const void* const* bytes,
                         const uint64_t* sizes) {
  if (!m || n < 0) return fail(lkrt::Status::error("null argument"));
  std::vector<lkrt::ExternalBytes> data;
  for (int i = 0; i < n; ++i) data.push_back({names[i], static_cast<const uint8_t*>(bytes[i]), sizes[i], nullptr});
  lkrt::Status s = lkrt::internalize(*m->m, data, true);
  return s ? 0 : fail(s);
}

int lk_model_num_inputs(const lk_model* m) { return m ? static_cast<int>(m->m->exec.args.size()) : -1; }

int lk_model_num_outputs(const lk_model* m) {
  if (!m || m->m->exec.ops.empty()) return -1;
  return static_cast<int>(m->m->exec.ops.back().operands.size());
}

int lk_model_input_is_mutable(const lk_model* m, int i) {
  return m && m->m->exec.isMutable(static_cast<size_t>(i)) ? 1 : 0;
}

void lk_model_free(lk_model* m) { delete m; }

char* lk_dim_canonical(const char* text) {
  lkrt::DimPool pool;
  std::string err;
  lkrt::Dim d = pool.parse(text ? text : "", err);
  if (!d) {
    lkh::setLastError(err);
    return nullptr;
  }
  return dupString(pool.str(d));
}

lk_model* lk_model_bake_init(const lk_model* m, int n_ext, const char* const* names, void* const* ptrs,
                             const uint64_t* sizes, const int* on_device, void* stream, uint64_t* stats) {
  if (!m || n_ext < 0) return failNull<lk_model>(lkrt::Status::error("null argument"));
  std::vector<lkrt::ExternalPtr> ext;
  for (int i = 0; i < n_ext; ++i) ext.push_back({names[i], ptrs[i], sizes[i], on_device[i] != 0});
  lkrt::Status st;
  lkrt::BakeStats bs;
  auto baked = lkrt::bakeInit(m->m, ext, static_cast<hipStream_t>(stream), &bs, st);
  if (!baked) return failNull<lk_model>(st);
  if (stats) {
    stats[0] = bs.baked;
    stats[1] = bs.bakedBytes;
    stats[2] = bs.initOpsBefore;
    stats[3] = bs.initOpsAfter;
  }
  return wrap(std::move(baked));
}

lk_exe* lk_exe_create(lk_model* m, int n_ext, const char* const* names, void* const* ptrs, const uint64_t* sizes,
                      const int* on_device, void* stream, int flags) {
  if (!m || n_ext < 0) return failNull<lk_exe>(lkrt::Status::error("null argument"));
  std::vector<lkrt::ExternalPtr> ext;
  for (int i = 0; i < n_ext; ++i) ext.push_back({names[i], ptrs[i], sizes[i], on_device[i] != 0});
  lkrt::Status st;
  const int streams = (flags >> 8) & 0xf;
  auto e = lkrt::Executable::create(m->m, ext, static_cast<hipStream_t>(stream), (flags & 1) != 0, st,
                                    streams ? streams : 1);
  if (!e) return failNull<lk_exe>(st);
  auto* w = new lk_exe;
  w->e = std::move(e);
  return w;
}

int lk_exe_run(lk_exe* e, int n_in, const lk_tensor* inputs, int max_out, lk_tensor* outputs, int* n_out,
               void* stream, int flags) {
  if (!e || n_in < 0 || (n_in && !inputs)) return fail(lkrt::Status::error("null argument"));
  std::vector<lkrt::TensorIn> in;
  for (int i = 0; i < n_in; ++i) {
    const lk_tensor& t = inputs[i];
    if (t.rank < 0 || t.rank > 8 || t.dtype < 0 || t.dtype > 8)
      return fail(lkrt::Status::error("input " + std::to_string(i) + ": bad rank or dtype"));
    in.push_back({t.data, std::vector<int64_t>(t.shape, t.shape + t.rank), static_cast<lkrt::DType>(t.dtype)});
  }
  std::vector<lkrt::TensorOut> out;
  lkrt::Status s = e->e->run(in, out, static_cast<hipStream_t>(stream), (flags & 1) != 0);
  if (!s) return fail(s);
  if (n_out) *n_out = static_cast<int>(out.size());
  if (static_cast<int>(out.size()) > max_out) return fail(lkrt::Status::error("too many outputs for the array"));
  for (size_t k = 0; k < out.size(); ++k) {
    if (out[k].shape.size() > 8) return fail(lkrt::Status::error("output rank above 8"));
    outputs[k].data = out[k].data;
    outputs[k].rank = static_cast<int32_t>(out[k].shape.size());
    outputs[k].dtype = static_cast<int32_t>(out[k].dtype);
    for (size_t j = 0; j < out[k].shape.size(); ++j) outputs[k].shape[j] = out[k].shape[j];
  }
  return 0;
}

int lk_exe_stats(const lk_exe* e, uint64_t* model_bytes, uint64_t* call_bytes, int* graphs, int* streams) {
  if (!e) return fail(lkrt::Status::error("null executable"));
  if (streams) *streams = e->e->lanesUsed();
  if (model_bytes) *model_bytes = e->e->modelArenaBytes();
  if (call_bytes) *call_bytes = e->e->callArenaBytes();
  if (graphs) *graphs = e->e->graphsCaptured();
  return 0;
}

void lk_exe_free(lk_exe* e) { delete e; }

}  // extern "C"

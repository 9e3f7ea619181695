// .lkm v2 model files: the reference's binary format (lariaus/lokinfer include/lokinfer/ir/binary.h:1-45,
// docs/impl-notes/design-ir.md §8). A 64-byte header {"LKM\0", u32 version, u64 meta offset / size, u64 data offset
// / size, reserved}, one metadata blob of LEB128 varints (zigzag for signed values), then the constants' bytes, each
// at a 16 KiB-aligned offset of the data section. Metadata order: symbols, dims (operands before the dims that use
// them), types, values, constants, then the init and exec regions; dims and types are numbered in first-use order.
//
// The codec is table-driven: a model is first flattened into plain tables (rows of numbers and strings that index
// each other), and ONE description of the table layout, `transfer`, is instantiated for a writing and a reading
// stream, so the two directions cannot drift apart. Reading then builds the model from the tables, rebuilding dims
// through the canonicalizing constructors and checking every cross-reference; constants point into the mapped file.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <unordered_map>

#include "ir.h"

namespace lkrt {

namespace {

constexpr uint32_t kVersion = 2;  // version 2 added the exec mutable-argument flags; version 1 files still load
constexpr uint64_t kHeaderBytes = 64;
constexpr uint64_t kConstAlign = 16384;
constexpr uint64_t kMaxCount = 1ull << 26;  // no table of a corrupt file may ask for more rows than this

uint64_t alignTo(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// ---- tables ------------------------------------------------------------------------------------------------------
struct DimRow {
  uint8_t kind = 0;
  int64_t value = 0;
  std::vector<uint64_t> args;
};
struct TypeRow {
  uint8_t kind = 0, dtype = 0;
  std::vector<uint64_t> shape;
};
struct ValueRow {
  uint64_t type = 0;
  std::string name;
};
struct ConstRow {
  std::string name;
  uint64_t type = 0, offset = 0, size = 0;
};
struct AttrRow {
  std::string name;
  uint8_t tag = 0;  // the AttrValue alternative
  uint8_t flag = 0;
  int64_t i = 0;
  double f = 0;
  std::string s;
  std::vector<int64_t> ints;
  std::vector<double> floats;
  uint64_t dim = 0;
};
struct OpRow {
  uint8_t kind = 0;
  std::string name;
  std::vector<uint64_t> operands, outs, results;
  std::vector<AttrRow> attrs;
  std::vector<uint8_t> data;
  std::vector<uint64_t> dims;
  std::vector<int64_t> ints;
  std::vector<uint64_t> symbols;
};
struct RegionRow {
  std::vector<uint64_t> args;
  std::vector<uint8_t> mutableFlags;
  std::vector<uint64_t> state;
  std::vector<OpRow> ops;
};
struct Tables {
  std::vector<std::string> symbols;
  std::vector<DimRow> dims;
  std::vector<TypeRow> types;
  std::vector<ValueRow> values;
  std::vector<ConstRow> consts;
  RegionRow regions[2];  // init, exec
};

// ---- streams -------------------------------------------------------------------------------------------------------
// Both have the same primitives; `transfer` below uses nothing else.
struct Put {
  static constexpr bool kReading = false;
  std::vector<uint8_t> out;
  bool ok() const { return true; }
  void var(uint64_t v) {
    do {
      out.push_back(static_cast<uint8_t>((v & 0x7f) | (v > 0x7f ? 0x80 : 0)));
      v >>= 7;
    } while (v);
  }
  void u(uint64_t& v) { var(v); }
  void i(int64_t& v) { var(static_cast<uint64_t>(v) << 1 ^ static_cast<uint64_t>(v >> 63)); }
  void b(uint8_t& v) { out.push_back(v); }
  void f(double& d) {
    uint64_t x;
    std::memcpy(&x, &d, 8);
    for (int k = 0; k < 64; k += 8) out.push_back(static_cast<uint8_t>(x >> k));
  }
  void s(std::string& v) {
    var(v.size());
    out.insert(out.end(), v.begin(), v.end());
  }
  void bytes(std::vector<uint8_t>& v) {
    var(v.size());
    out.insert(out.end(), v.begin(), v.end());
  }
  template <class T, class F>
  void list(std::vector<T>& v, F&& each) {
    var(v.size());
    for (T& x : v) each(x);
  }
};

struct Get {
  static constexpr bool kReading = true;
  const uint8_t* p;
  const uint8_t* end;
  bool good = true;
  bool ok() const { return good; }
  void fail() {
    good = false;
    p = end;
  }
  uint64_t var() {
    uint64_t v = 0;
    for (int shift = 0; shift < 64 && p < end; shift += 7) {
      const uint8_t c = *p++;
      v |= static_cast<uint64_t>(c & 0x7f) << shift;
      if (!(c & 0x80)) return v;
    }
    fail();
    return 0;
  }
  void u(uint64_t& v) { v = var(); }
  void i(int64_t& v) {
    const uint64_t z = var();
    v = static_cast<int64_t>(z >> 1) ^ -static_cast<int64_t>(z & 1);
  }
  void b(uint8_t& v) {
    if (p < end) v = *p++;
    else fail();
  }
  void f(double& d) {
    uint64_t x = 0;
    if (end - p < 8) return fail();
    for (int k = 0; k < 8; ++k) x |= static_cast<uint64_t>(*p++) << (8 * k);
    std::memcpy(&d, &x, 8);
  }
  void s(std::string& v) {
    const uint64_t n = var();
    if (static_cast<uint64_t>(end - p) < n) return fail();
    v.assign(reinterpret_cast<const char*>(p), n);
    p += n;
  }
  void bytes(std::vector<uint8_t>& v) {
    const uint64_t n = var();
    if (static_cast<uint64_t>(end - p) < n) return fail();
    v.assign(p, p + n);
    p += n;
  }
  template <class T, class F>
  void list(std::vector<T>& v, F&& each) {
    const uint64_t n = var();
    if (n > kMaxCount) return fail();
    v.clear();
    for (uint64_t k = 0; k < n && good; ++k) each(v.emplace_back());
  }
};

// ---- the layout (one description for both directions) ----------------------------------------------------------------
template <class IO>
void transferAttr(IO& io, AttrRow& a) {
  io.s(a.name);
  io.b(a.tag);
  switch (a.tag) {
    case 0: io.b(a.flag); break;
    case 1: io.i(a.i); break;
    case 2: io.f(a.f); break;
    case 3: io.s(a.s); break;
    case 4: io.list(a.ints, [&](int64_t& x) { io.i(x); }); break;
    case 5: io.list(a.floats, [&](double& x) { io.f(x); }); break;
    case 6: io.u(a.dim); break;
    default:
      if constexpr (IO::kReading) io.fail();
  }
}

template <class IO>
void transferRegion(IO& io, RegionRow& r, uint32_t version) {
  auto ids = [&](std::vector<uint64_t>& v) { io.list(v, [&](uint64_t& x) { io.u(x); }); };
  ids(r.args);
  if (version >= 2) io.list(r.mutableFlags, [&](uint8_t& x) { io.b(x); });
  ids(r.state);
  io.list(r.ops, [&](OpRow& op) {
    io.b(op.kind);
    io.s(op.name);
    ids(op.operands);
    ids(op.outs);
    ids(op.results);
    io.list(op.attrs, [&](AttrRow& a) { transferAttr(io, a); });
    io.bytes(op.data);
    ids(op.dims);
    io.list(op.ints, [&](int64_t& x) { io.i(x); });
    ids(op.symbols);
  });
}

template <class IO>
void transfer(IO& io, Tables& t, uint32_t version) {
  io.list(t.symbols, [&](std::string& s) { io.s(s); });
  io.list(t.dims, [&](DimRow& d) {
    io.b(d.kind);
    io.i(d.value);
    io.list(d.args, [&](uint64_t& x) { io.u(x); });
  });
  io.list(t.types, [&](TypeRow& ty) {
    io.b(ty.kind);
    io.b(ty.dtype);
    io.list(ty.shape, [&](uint64_t& x) { io.u(x); });
  });
  io.list(t.values, [&](ValueRow& v) {
    io.u(v.type);
    io.s(v.name);
  });
  io.list(t.consts, [&](ConstRow& c) {
    io.s(c.name);
    io.u(c.type);
    io.u(c.offset);
    io.u(c.size);
  });
  for (RegionRow& r : t.regions) transferRegion(io, r, version);
}

// ---- model -> tables ---------------------------------------------------------------------------------------------------
class Flattener {
 public:
  explicit Flattener(const Model& m) : m_(m) {}

  Status run(Tables& t) {
    // numbering: value types (with their dims), constant types, then the dims ops and dim attributes carry
    for (ValueId v = 0; v < m_.numValues(); ++v) typeIndex(m_.typeOf(v));
    for (const Constant& c : m_.constants) typeIndex(c.type);
    for (const Region* r : {&m_.init, &m_.exec})
      for (const Op& op : r->ops) {
        for (Dim d : op.dims) dimIndex(d);
        for (const NamedAttr& a : op.attrs)
          if (const Dim* d = std::get_if<Dim>(&a.value)) dimIndex(*d);
      }
    const DimPool& dp = m_.dims();
    for (size_t k = 0; k < dp.numSymbols(); ++k) t.symbols.push_back(dp.symbolName(static_cast<int64_t>(k)));
    for (Dim d : dimOrder_) {
      DimRow row{static_cast<uint8_t>(d->kind), d->value, {}};
      for (Dim a : d->args) row.args.push_back(dimNo_.at(a));
      t.dims.push_back(std::move(row));
    }
    for (Type ty : typeOrder_) {
      TypeRow row{static_cast<uint8_t>(ty->kind), static_cast<uint8_t>(ty->dtype), {}};
      for (Dim d : ty->shape) row.shape.push_back(dimNo_.at(d));
      t.types.push_back(std::move(row));
    }
    for (ValueId v = 0; v < m_.numValues(); ++v) t.values.push_back({typeNo_.at(m_.typeOf(v)), m_.nameOf(v)});
    uint64_t at = 0;
    for (const Constant& c : m_.constants) {
      if (!c.bytes && c.size) return Status::error("constant '" + c.name + "' has no data");
      t.consts.push_back({c.name, typeNo_.at(c.type), at, c.size});
      at = alignTo(at + c.size, kConstAlign);
    }
    flattenRegion(m_.init, t.regions[0]);
    flattenRegion(m_.exec, t.regions[1]);
    return Status();
  }

 private:
  uint64_t dimIndex(Dim d) {
    if (auto it = dimNo_.find(d); it != dimNo_.end()) return it->second;
    for (Dim a : d->args) dimIndex(a);
    dimOrder_.push_back(d);
    return dimNo_[d] = dimOrder_.size() - 1;
  }
  uint64_t typeIndex(Type t) {
    if (auto it = typeNo_.find(t); it != typeNo_.end()) return it->second;
    for (Dim d : t->shape) dimIndex(d);
    typeOrder_.push_back(t);
    return typeNo_[t] = typeOrder_.size() - 1;
  }
  static std::vector<uint64_t> widen(const std::vector<ValueId>& v) { return {v.begin(), v.end()}; }
  void flattenRegion(const Region& r, RegionRow& out) {
    out.args = widen(r.args);
    out.mutableFlags = r.mutableArgs;
    out.state = widen(r.state);
    for (const Op& op : r.ops) {
      OpRow row;
      row.kind = static_cast<uint8_t>(op.kind);
      row.name = op.name;
      row.operands = widen(op.operands);
      row.outs = widen(op.outs);
      row.results = widen(op.results);
      for (const NamedAttr& a : op.attrs) {
        AttrRow ar;
        ar.name = a.name;
        ar.tag = static_cast<uint8_t>(a.value.index());
        std::visit(
            [&](const auto& x) {
              using T = std::decay_t<decltype(x)>;
              if constexpr (std::is_same_v<T, bool>) ar.flag = x ? 1 : 0;
              else if constexpr (std::is_same_v<T, int64_t>) ar.i = x;
              else if constexpr (std::is_same_v<T, double>) ar.f = x;
              else if constexpr (std::is_same_v<T, std::string>) ar.s = x;
              else if constexpr (std::is_same_v<T, Ints>) ar.ints = x;
              else if constexpr (std::is_same_v<T, Floats>) ar.floats = x;
              else ar.dim = dimNo_.at(x);
            },
            a.value);
        row.attrs.push_back(std::move(ar));
      }
      row.data = op.data;
      for (Dim d : op.dims) row.dims.push_back(dimNo_.at(d));
      row.ints = op.ints;
      for (int64_t s : op.symbols) row.symbols.push_back(static_cast<uint64_t>(s));
      out.ops.push_back(std::move(row));
    }
  }

  const Model& m_;
  std::vector<Dim> dimOrder_;
  std::unordered_map<Dim, uint64_t> dimNo_;
  std::vector<Type> typeOrder_;
  std::unordered_map<Type, uint64_t> typeNo_;
};

// ---- tables -> model ---------------------------------------------------------------------------------------------------
class Builder {
 public:
  Builder(const Tables& t, const uint8_t* data, uint64_t dataSize, std::shared_ptr<const void> owner)
      : t_(t), data_(data), dataSize_(dataSize), owner_(std::move(owner)), m_(std::make_unique<Model>()) {}

  std::unique_ptr<Model> run(std::string& err) {
    if (!symbols() || !dims() || !types() || !values() || !constants() || !region(t_.regions[0], m_->init) ||
        !region(t_.regions[1], m_->exec)) {
      err = err_;
      return nullptr;
    }
    return std::move(m_);
  }

 private:
  bool bad(std::string msg) {
    err_ = std::move(msg);
    return false;
  }
  bool symbols() {
    for (const std::string& s : t_.symbols) sym_.push_back(m_->dims().sym(s)->value);
    return true;
  }
  bool dims() {
    DimPool& dp = m_->dims();
    for (const DimRow& r : t_.dims) {
      std::vector<Dim> a;
      for (uint64_t j : r.args) {
        if (j >= dim_.size()) return bad("bad dim reference");
        a.push_back(dim_[j]);
      }
      if (r.kind > static_cast<uint8_t>(DimKind::Max)) return bad("bad dim kind");
      const DimKind k = static_cast<DimKind>(r.kind);
      Dim d = nullptr;  // stored nodes are canonical; rebuilding them through the constructors returns the same form
      if (k == DimKind::Const) {
        d = dp.constant(r.value);
      } else if (k == DimKind::Sym) {
        if (r.value < 0 || static_cast<uint64_t>(r.value) >= sym_.size()) return bad("bad symbol");
        d = dp.sym(dp.symbolName(sym_[static_cast<size_t>(r.value)]));
      } else if (k == DimKind::Add || k == DimKind::Mul) {
        if (a.empty()) return bad("empty n-ary dim");
        d = a[0];
        for (size_t q = 1; q < a.size(); ++q) d = k == DimKind::Add ? dp.add(d, a[q]) : dp.mul(d, a[q]);
      } else {
        if (a.size() != 2) return bad("binary dim needs 2 operands");
        const bool divides = k == DimKind::FloorDiv || k == DimKind::CeilDiv || k == DimKind::Mod;
        if (divides && a[1]->isConst(0)) return bad("division by zero in a dim");
        switch (k) {
          case DimKind::FloorDiv: d = dp.floorDiv(a[0], a[1]); break;
          case DimKind::CeilDiv: d = dp.ceilDiv(a[0], a[1]); break;
          case DimKind::Mod: d = dp.mod(a[0], a[1]); break;
          case DimKind::Min: d = dp.min(a[0], a[1]); break;
          default: d = dp.max(a[0], a[1]);
        }
      }
      dim_.push_back(d);
    }
    return true;
  }
  bool types() {
    for (const TypeRow& r : t_.types) {
      if (r.kind > static_cast<uint8_t>(TypeKind::Buffer) || r.dtype > static_cast<uint8_t>(DType::Bool) ||
          r.shape.size() > 64)
        return bad("bad type");
      std::vector<Dim> shape;
      for (uint64_t j : r.shape) {
        if (j >= dim_.size()) return bad("bad dim reference in type");
        shape.push_back(dim_[j]);
      }
      type_.push_back(m_->types().get(static_cast<TypeKind>(r.kind), static_cast<DType>(r.dtype), shape));
    }
    return true;
  }
  bool values() {
    for (const ValueRow& v : t_.values) {
      if (v.type >= type_.size()) return bad("bad type reference");
      m_->newValue(type_[v.type], v.name);
    }
    return true;
  }
  bool constants() {
    for (const ConstRow& r : t_.consts) {
      if (r.type >= type_.size() || r.offset > dataSize_ || r.size > dataSize_ - r.offset)
        return bad("bad constant '" + r.name + "'");
      Constant c;
      c.name = r.name;
      c.type = type_[r.type];
      c.size = r.size;
      // a statically shaped constant's byte count must be its type's
      uint64_t want = dtypeSize(c.type->dtype);
      bool known = true;
      for (Dim d : c.type->shape) {
        known = known && d->isConst() && d->value >= 0 && (d->value == 0 || want <= UINT64_MAX / d->value);
        if (known) want *= static_cast<uint64_t>(d->value);
      }
      if (known && want != c.size) return bad("constant '" + c.name + "' size doesn't match its type");
      c.bytes = data_ + r.offset;
      c.owner = owner_;
      m_->addConstant(std::move(c));
    }
    return true;
  }
  bool ids(const std::vector<uint64_t>& in, std::vector<ValueId>& out) {
    for (uint64_t v : in) {
      if (v >= m_->numValues()) return bad("bad value reference");
      out.push_back(static_cast<ValueId>(v));
    }
    return true;
  }
  bool region(const RegionRow& r, Region& reg) {
    if (!ids(r.args, reg.args) || !ids(r.state, reg.state)) return false;
    if (!r.mutableFlags.empty() && r.mutableFlags.size() != r.args.size()) return bad("bad mutable-arg flags");
    for (uint8_t f : r.mutableFlags) reg.mutableArgs.push_back(f != 0);
    for (const OpRow& o : r.ops) {
      if (o.kind > static_cast<uint8_t>(OpKind::Return)) return bad("bad op kind");
      Op op;
      op.kind = static_cast<OpKind>(o.kind);
      op.name = o.name;
      if (!ids(o.operands, op.operands) || !ids(o.outs, op.outs) || !ids(o.results, op.results)) return false;
      for (const AttrRow& a : o.attrs) {
        NamedAttr na{a.name, false};
        switch (a.tag) {
          case 0: na.value = a.flag != 0; break;
          case 1: na.value = a.i; break;
          case 2: na.value = a.f; break;
          case 3: na.value = a.s; break;
          case 4: na.value = a.ints; break;
          case 5: na.value = a.floats; break;
          default:
            if (a.dim >= dim_.size()) return bad("bad dim attribute");
            na.value = dim_[a.dim];
        }
        op.attrs.push_back(std::move(na));
      }
      op.data = o.data;
      for (uint64_t j : o.dims) {
        if (j >= dim_.size()) return bad("bad dim reference in op");
        op.dims.push_back(dim_[j]);
      }
      op.ints = o.ints;
      for (uint64_t s : o.symbols) {
        if (s >= sym_.size()) return bad("bad symbol reference");
        op.symbols.push_back(sym_[s]);
      }
      reg.ops.push_back(std::move(op));
    }
    return true;
  }

  const Tables& t_;
  const uint8_t* data_;
  uint64_t dataSize_;
  std::shared_ptr<const void> owner_;
  std::unique_ptr<Model> m_;
  std::vector<int64_t> sym_;
  std::vector<Dim> dim_;
  std::vector<Type> type_;
  std::string err_;
};

// little-endian header fields
template <class T>
void storeLe(uint8_t* p, T v) {
  for (size_t k = 0; k < sizeof(T); ++k) p[k] = static_cast<uint8_t>(v >> (8 * k));
}
template <class T>
T loadLe(const uint8_t* p) {
  T v = 0;
  for (size_t k = 0; k < sizeof(T); ++k) v |= static_cast<T>(p[k]) << (8 * k);
  return v;
}

}  // namespace

std::vector<uint8_t> writeLkm(const Model& m, Status& st) {
  for (const Region* r : {&m.init, &m.exec})
    for (const Op& op : r->ops)
      if (op.kind == OpKind::ConstExternal) {
        st = Status::error("lkm: external constant '" + op.name + "' must be internalized before export");
        return {};
      }
  Tables t;
  if (st = Flattener(m).run(t); !st) return {};
  Put meta;
  transfer(meta, t, kVersion);
  const uint64_t dataOff = alignTo(kHeaderBytes + meta.out.size(), kConstAlign);
  uint64_t dataSize = 0;
  for (const ConstRow& c : t.consts) dataSize = std::max(dataSize, c.offset + c.size);
  std::vector<uint8_t> file(dataOff + dataSize, 0);
  std::memcpy(file.data(), "LKM\0", 4);
  storeLe<uint32_t>(file.data() + 4, kVersion);
  storeLe<uint64_t>(file.data() + 8, kHeaderBytes);
  storeLe<uint64_t>(file.data() + 16, meta.out.size());
  storeLe<uint64_t>(file.data() + 24, dataOff);
  storeLe<uint64_t>(file.data() + 32, dataSize);
  std::copy(meta.out.begin(), meta.out.end(), file.begin() + kHeaderBytes);
  for (size_t k = 0; k < t.consts.size(); ++k)
    if (t.consts[k].size) std::memcpy(file.data() + dataOff + t.consts[k].offset, m.constants[k].bytes, t.consts[k].size);
  return file;
}

std::unique_ptr<Model> readLkm(const uint8_t* base, size_t size, std::shared_ptr<const void> owner, Status& st) {
  auto fail = [&](const std::string& msg) -> std::unique_ptr<Model> {
    st = Status::error("lkm: " + msg);
    return nullptr;
  };
  if (size < kHeaderBytes) return fail("file too small");
  if (std::memcmp(base, "LKM\0", 4) != 0) return fail("bad magic");
  const uint32_t version = loadLe<uint32_t>(base + 4);
  if (version != 1 && version != kVersion) return fail("unsupported version " + std::to_string(version));
  const uint64_t metaOff = loadLe<uint64_t>(base + 8), metaSize = loadLe<uint64_t>(base + 16);
  const uint64_t dataOff = loadLe<uint64_t>(base + 24), dataSize = loadLe<uint64_t>(base + 32);
  if (metaOff > size || metaSize > size - metaOff || dataOff > size || dataSize > size - dataOff)
    return fail("truncated file");
  Tables t;
  Get in{base + metaOff, base + metaOff + metaSize};
  transfer(in, t, version);
  if (!in.ok()) return fail("corrupt metadata");
  std::string err;
  auto m = Builder(t, base + dataOff, dataSize, std::move(owner)).run(err);
  if (!m) return fail(err);
  st = Status();
  return m;
}

Status writeLkmFile(const Model& m, const std::string& path) {
  Status st;
  const std::vector<uint8_t> bytes = writeLkm(m, st);
  if (!st) return st;
  std::FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) return Status::error("cannot open " + path + " for writing");
  const bool wrote = std::fwrite(bytes.data(), 1, bytes.size(), f) == bytes.size();
  if (std::fclose(f) != 0 || !wrote) return Status::error("failed writing " + path);
  return Status();
}

std::unique_ptr<Model> readLkmFile(const std::string& path, Status& st) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) {
    st = Status::error("cannot open " + path);
    return nullptr;
  }
  struct stat info {};
  const bool statOk = ::fstat(fd, &info) == 0;
  if (!statOk || info.st_size <= 0) {
    ::close(fd);
    st = Status::error(statOk ? "lkm: file too small" : "cannot stat " + path);
    return nullptr;
  }
  const size_t size = static_cast<size_t>(info.st_size);
  void* map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) {
    st = Status::error("cannot mmap " + path);
    return nullptr;
  }
  std::shared_ptr<const void> owner(map, [size](const void* q) { ::munmap(const_cast<void*>(q), size); });
  return readLkm(static_cast<const uint8_t*>(map), size, owner, st);
}

}  // namespace lkrt

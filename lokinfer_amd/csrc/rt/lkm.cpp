// .lkm v2 model files (the reference's binary format, lariaus/lokinfer include/lokinfer/ir/binary.h:1-45 and
// docs/impl-notes/design-ir.md §8): a 64-byte header {"LKM\0", u32 version, u64 meta offset / size, u64 data
// offset / size, 24 reserved bytes}, one metadata blob of LEB128 varints (zigzag for signed values), then the
// constants' bytes, each 16 KiB-aligned within the data section. Metadata order: symbols, dims (operands first),
// types, values, constants, then the init and exec regions. Dims and types are numbered in first-use order.
// Reading maps the file and points every constant into the mapping (no copy).
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

constexpr uint32_t kLkmVersion = 2;  // version 2 added the exec mutable-argument flags (version 1 is still read)
constexpr size_t kHeader = 64;
constexpr uint64_t kDataAlign = 16384;

uint64_t roundUp(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// ---- encoding --------------------------------------------------------------------------------------------------
struct Sink {
  std::vector<uint8_t> b;
  void byte(uint8_t v) { b.push_back(v); }
  void u(uint64_t v) {
    for (; v >= 0x80; v >>= 7) b.push_back(static_cast<uint8_t>(v | 0x80));
    b.push_back(static_cast<uint8_t>(v));
  }
  void s(int64_t v) { u((static_cast<uint64_t>(v) << 1) ^ static_cast<uint64_t>(v >> 63)); }
  void f(double d) {
    uint64_t x;
    std::memcpy(&x, &d, 8);
    for (int i = 0; i < 8; ++i) b.push_back(static_cast<uint8_t>(x >> (8 * i)));
  }
  void str(const std::string& v) {
    u(v.size());
    b.insert(b.end(), v.begin(), v.end());
  }
  void ids(const std::vector<ValueId>& v) {
    u(v.size());
    for (ValueId x : v) u(x);
  }
};

class Encoder {
 public:
  explicit Encoder(const Model& m) : m_(m) {}

  // Appends the metadata to `out`; `offsets` receives each constant's offset within the data section.
  Status run(Sink& out, std::vector<uint64_t>& offsets) {
    for (ValueId v = 0; v < m_.numValues(); ++v) typeNo(m_.typeOf(v));
    for (const Constant& c : m_.constants) typeNo(c.type);
    for (const Region* r : {&m_.init, &m_.exec})
      for (const Op& op : r->ops) {
        for (Dim d : op.dims) dimNo(d);
        for (const NamedAttr& a : op.attrs)
          if (a.value.index() == 6) dimNo(std::get<Dim>(a.value));
      }
    const DimPool& dp = m_.dims();
    out.u(dp.numSymbols());
    for (size_t i = 0; i < dp.numSymbols(); ++i) out.str(dp.symbolName(static_cast<int64_t>(i)));
    out.u(dimList_.size());
    for (Dim d : dimList_) {
      out.byte(static_cast<uint8_t>(d->kind));
      out.s(d->value);
      out.u(d->args.size());
      for (Dim a : d->args) out.u(dimIdx_.at(a));
    }
    out.u(typeList_.size());
    for (Type t : typeList_) {
      out.byte(static_cast<uint8_t>(t->kind));
      out.byte(static_cast<uint8_t>(t->dtype));
      out.u(t->shape.size());
      for (Dim d : t->shape) out.u(dimIdx_.at(d));
    }
    out.u(m_.numValues());
    for (ValueId v = 0; v < m_.numValues(); ++v) {
      out.u(typeIdx_.at(m_.typeOf(v)));
      out.str(m_.nameOf(v));
    }
    uint64_t off = 0;
    out.u(m_.constants.size());
    for (const Constant& c : m_.constants) {
      if (!c.bytes && c.size) return Status::error("constant '" + c.name + "' has no data");
      out.str(c.name);
      out.u(typeIdx_.at(c.type));
      out.u(off);
      out.u(c.size);
      offsets.push_back(off);
      off = roundUp(off + c.size, kDataAlign);
    }
    for (const Region* r : {&m_.init, &m_.exec}) region(out, *r);
    return Status();
  }

 private:
  size_t dimNo(Dim d) {
    auto it = dimIdx_.find(d);
    if (it != dimIdx_.end()) return it->second;
    for (Dim a : d->args) dimNo(a);
    dimIdx_[d] = dimList_.size();
    dimList_.push_back(d);
    return dimList_.size() - 1;
  }
  size_t typeNo(Type t) {
    auto it = typeIdx_.find(t);
    if (it != typeIdx_.end()) return it->second;
    for (Dim d : t->shape) dimNo(d);
    typeIdx_[t] = typeList_.size();
    typeList_.push_back(t);
    return typeList_.size() - 1;
  }
  void region(Sink& out, const Region& r) {
    out.ids(r.args);
    out.u(r.mutableArgs.size());
    for (uint8_t f : r.mutableArgs) out.byte(f);
    out.ids(r.state);
    out.u(r.ops.size());
    for (const Op& op : r.ops) {
      out.byte(static_cast<uint8_t>(op.kind));
      out.str(op.name);
      out.ids(op.operands);
      out.ids(op.outs);
      out.ids(op.results);
      out.u(op.attrs.size());
      for (const NamedAttr& a : op.attrs) {
        out.str(a.name);
        out.byte(static_cast<uint8_t>(a.value.index()));
        switch (a.value.index()) {
          case 0: out.byte(std::get<bool>(a.value) ? 1 : 0); break;
          case 1: out.s(std::get<int64_t>(a.value)); break;
          case 2: out.f(std::get<double>(a.value)); break;
          case 3: out.str(std::get<std::string>(a.value)); break;
          case 4:
            out.u(std::get<Ints>(a.value).size());
            for (int64_t x : std::get<Ints>(a.value)) out.s(x);
            break;
          case 5:
            out.u(std::get<Floats>(a.value).size());
            for (double x : std::get<Floats>(a.value)) out.f(x);
            break;
          default: out.u(dimIdx_.at(std::get<Dim>(a.value)));
        }
      }
      out.u(op.data.size());
      out.b.insert(out.b.end(), op.data.begin(), op.data.end());
      out.u(op.dims.size());
      for (Dim d : op.dims) out.u(dimIdx_.at(d));
      out.u(op.ints.size());
      for (int64_t x : op.ints) out.s(x);
      out.u(op.symbols.size());
      for (int64_t x : op.symbols) out.u(static_cast<uint64_t>(x));
    }
  }

  const Model& m_;
  std::vector<Dim> dimList_;
  std::unordered_map<Dim, size_t> dimIdx_;
  std::vector<Type> typeList_;
  std::unordered_map<Type, size_t> typeIdx_;
};

void putU32(uint8_t* p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = static_cast<uint8_t>(v >> (8 * i));
}
void putU64(uint8_t* p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = static_cast<uint8_t>(v >> (8 * i));
}
uint32_t getU32(const uint8_t* p) {
  uint32_t v = 0;
  for (int i = 0; i < 4; ++i) v |= static_cast<uint32_t>(p[i]) << (8 * i);
  return v;
}
uint64_t getU64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= static_cast<uint64_t>(p[i]) << (8 * i);
  return v;
}

// ---- decoding --------------------------------------------------------------------------------------------------
class Source {
 public:
  Source(const uint8_t* p, size_t n) : p_(p), end_(p + n) {}
  bool ok() const { return ok_; }
  uint8_t byte() {
    if (p_ >= end_) return bad();
    return *p_++;
  }
  uint64_t u() {
    uint64_t v = 0;
    for (int sh = 0; sh < 64; sh += 7) {
      if (p_ >= end_) return bad();
      const uint8_t b = *p_++;
      v |= static_cast<uint64_t>(b & 0x7f) << sh;
      if (!(b & 0x80)) return v;
    }
    return bad();
  }
  int64_t s() {
    const uint64_t x = u();
    return static_cast<int64_t>(x >> 1) ^ -static_cast<int64_t>(x & 1);
  }
  double f() {
    if (end_ - p_ < 8) return bad();
    uint64_t x = getU64(p_);
    p_ += 8;
    double d;
    std::memcpy(&d, &x, 8);
    return d;
  }
  std::string str() {
    const uint64_t n = u();
    if (static_cast<uint64_t>(end_ - p_) < n) return bad(), std::string();
    std::string v(reinterpret_cast<const char*>(p_), n);
    p_ += n;
    return v;
  }
  std::vector<uint8_t> bytes() {
    const uint64_t n = u();
    if (static_cast<uint64_t>(end_ - p_) < n) return bad(), std::vector<uint8_t>();
    std::vector<uint8_t> v(p_, p_ + n);
    p_ += n;
    return v;
  }
  uint64_t count(uint64_t max = 1ull << 26) {  // bounded: a corrupt file must not allocate without limit
    const uint64_t n = u();
    return n > max ? bad() : n;
  }

 private:
  uint8_t bad() {
    ok_ = false;
    p_ = end_;
    return 0;
  }
  const uint8_t* p_;
  const uint8_t* end_;
  bool ok_ = true;
};

}  // namespace

std::vector<uint8_t> writeLkm(const Model& m, Status& st) {
  for (const Region* r : {&m.init, &m.exec})
    for (const Op& op : r->ops)
      if (op.kind == OpKind::ConstExternal) {
        st = Status::error("lkm: external constant '" + op.name + "' must be internalized before export");
        return {};
      }
  Sink meta;
  std::vector<uint64_t> offsets;
  st = Encoder(m).run(meta, offsets);
  if (!st) return {};
  const uint64_t dataOffset = roundUp(kHeader + meta.b.size(), kDataAlign);
  uint64_t dataSize = 0;
  for (size_t i = 0; i < offsets.size(); ++i) dataSize = std::max<uint64_t>(dataSize, offsets[i] + m.constants[i].size);
  std::vector<uint8_t> out(dataOffset + dataSize, 0);
  std::memcpy(out.data(), "LKM\0", 4);
  putU32(out.data() + 4, kLkmVersion);
  putU64(out.data() + 8, kHeader);
  putU64(out.data() + 16, meta.b.size());
  putU64(out.data() + 24, dataOffset);
  putU64(out.data() + 32, dataSize);
  std::memcpy(out.data() + kHeader, meta.b.data(), meta.b.size());
  for (size_t i = 0; i < offsets.size(); ++i)
    if (m.constants[i].size) std::memcpy(out.data() + dataOffset + offsets[i], m.constants[i].bytes, m.constants[i].size);
  return out;
}

std::unique_ptr<Model> readLkm(const uint8_t* base, size_t size, std::shared_ptr<const void> owner, Status& st) {
  auto fail = [&](const std::string& msg) {
    st = Status::error("lkm: " + msg);
    return nullptr;
  };
  if (size < kHeader) return fail("file too small");
  if (std::memcmp(base, "LKM\0", 4) != 0) return fail("bad magic");
  const uint32_t version = getU32(base + 4);
  if (version != 1 && version != kLkmVersion) return fail("unsupported version " + std::to_string(version));
  const uint64_t metaOff = getU64(base + 8), metaSize = getU64(base + 16);
  const uint64_t dataOff = getU64(base + 24), dataSize = getU64(base + 32);
  if (metaOff > size || metaSize > size - metaOff || dataOff > size || dataSize > size - dataOff)
    return fail("truncated file");
  Source r(base + metaOff, metaSize);
  auto m = std::make_unique<Model>();
  DimPool& dp = m->dims();
  std::vector<int64_t> symOf;  // file symbol index -> pool symbol id
  for (uint64_t i = 0, n = r.count(); i < n && r.ok(); ++i) symOf.push_back(dp.sym(r.str())->value);
  std::vector<Dim> dimOf;
  for (uint64_t i = 0, n = r.count(); i < n && r.ok(); ++i) {
    const uint8_t kindByte = r.byte();
    const int64_t value = r.s();
    std::vector<Dim> args;
    for (uint64_t k = 0, na = r.count(); k < na && r.ok(); ++k) {
      const uint64_t j = r.u();
      if (j >= dimOf.size()) return fail("bad dim reference");
      args.push_back(dimOf[j]);
    }
    if (!r.ok()) break;
    if (kindByte > static_cast<uint8_t>(DimKind::Max)) return fail("bad dim kind");
    const DimKind kind = static_cast<DimKind>(kindByte);
    Dim d = nullptr;  // rebuilt through the canonicalizing constructors (stored nodes are canonical)
    switch (kind) {
      case DimKind::Const: d = dp.constant(value); break;
      case DimKind::Sym:
        if (value < 0 || static_cast<size_t>(value) >= symOf.size()) return fail("bad symbol");
        d = dp.sym(dp.symbolName(symOf[static_cast<size_t>(value)]));
        break;
      case DimKind::Add:
      case DimKind::Mul:
        if (args.empty()) return fail("empty n-ary dim");
        d = args[0];
        for (size_t k = 1; k < args.size(); ++k) d = kind == DimKind::Add ? dp.add(d, args[k]) : dp.mul(d, args[k]);
        break;
      default:
        if (args.size() != 2) return fail("binary dim needs 2 operands");
        if ((kind == DimKind::FloorDiv || kind == DimKind::CeilDiv || kind == DimKind::Mod) && args[1]->isConst(0))
          return fail("division by zero in a dim");
        d = kind == DimKind::FloorDiv ? dp.floorDiv(args[0], args[1])
            : kind == DimKind::CeilDiv ? dp.ceilDiv(args[0], args[1])
            : kind == DimKind::Mod     ? dp.mod(args[0], args[1])
            : kind == DimKind::Min     ? dp.min(args[0], args[1])
                                       : dp.max(args[0], args[1]);
    }
    dimOf.push_back(d);
  }
  std::vector<Type> typeOf;
  for (uint64_t i = 0, n = r.count(); i < n && r.ok(); ++i) {
    const uint8_t kb = r.byte(), db = r.byte();
    if (kb > static_cast<uint8_t>(TypeKind::Buffer) || db > static_cast<uint8_t>(DType::Bool)) return fail("bad type");
    std::vector<Dim> shape;
    for (uint64_t k = 0, rank = r.count(64); k < rank && r.ok(); ++k) {
      const uint64_t j = r.u();
      if (j >= dimOf.size()) return fail("bad dim reference in type");
      shape.push_back(dimOf[j]);
    }
    typeOf.push_back(m->types().get(static_cast<TypeKind>(kb), static_cast<DType>(db), shape));
  }
  for (uint64_t i = 0, n = r.count(); i < n && r.ok(); ++i) {
    const uint64_t t = r.u();
    std::string name = r.str();
    if (t >= typeOf.size()) return fail("bad type reference");
    m->newValue(typeOf[t], std::move(name));
  }
  for (uint64_t i = 0, n = r.count(); i < n && r.ok(); ++i) {
    Constant c;
    c.name = r.str();
    const uint64_t t = r.u(), off = r.u();
    c.size = r.u();
    if (!r.ok()) break;
    if (t >= typeOf.size() || off > dataSize || c.size > dataSize - off) return fail("bad constant '" + c.name + "'");
    c.type = typeOf[t];
    uint64_t bytes = dtypeSize(c.type->dtype);
    bool known = true;
    for (Dim d : c.type->shape) {
      if (!d->isConst() || d->value < 0 || (d->value && bytes > UINT64_MAX / static_cast<uint64_t>(d->value))) {
        known = false;
        break;
      }
      bytes *= static_cast<uint64_t>(d->value);
    }
    if (known && bytes != c.size) return fail("constant '" + c.name + "' size doesn't match its type");
    c.bytes = base + dataOff + off;
    c.owner = owner;
    m->addConstant(std::move(c));
  }
  auto ids = [&](std::vector<ValueId>& v) {
    for (uint64_t k = 0, n = r.count(); k < n && r.ok(); ++k) v.push_back(static_cast<ValueId>(r.u()));
  };
  for (Region* reg : {&m->init, &m->exec}) {
    ids(reg->args);
    if (version >= 2) {
      const uint64_t n = r.count();
      if (n != 0 && n != reg->args.size()) return fail("bad mutable-arg flags");
      for (uint64_t k = 0; k < n && r.ok(); ++k) reg->mutableArgs.push_back(r.byte() != 0);
    }
    ids(reg->state);
    for (uint64_t i = 0, n = r.count(); i < n && r.ok(); ++i) {
      Op op;
      const uint8_t kb = r.byte();
      if (kb > static_cast<uint8_t>(OpKind::Return)) return fail("bad op kind");
      op.kind = static_cast<OpKind>(kb);
      op.name = r.str();
      ids(op.operands);
      ids(op.outs);
      ids(op.results);
      for (uint64_t k = 0, na = r.count(); k < na && r.ok(); ++k) {
        NamedAttr a;
        a.name = r.str();
        switch (r.byte()) {
          case 0: a.value = r.byte() != 0; break;
          case 1: a.value = r.s(); break;
          case 2: a.value = r.f(); break;
          case 3: a.value = r.str(); break;
          case 4: {
            Ints v;
            for (uint64_t j = 0, nv = r.count(); j < nv && r.ok(); ++j) v.push_back(r.s());
            a.value = std::move(v);
            break;
          }
          case 5: {
            Floats v;
            for (uint64_t j = 0, nv = r.count(); j < nv && r.ok(); ++j) v.push_back(r.f());
            a.value = std::move(v);
            break;
          }
          case 6: {
            const uint64_t j = r.u();
            if (j >= dimOf.size()) return fail("bad dim attribute");
            a.value = dimOf[j];
            break;
          }
          default:
            if (r.ok()) return fail("bad attribute tag");
        }
        op.attrs.push_back(std::move(a));
      }
      op.data = r.bytes();
      for (uint64_t k = 0, nd = r.count(); k < nd && r.ok(); ++k) {
        const uint64_t j = r.u();
        if (j >= dimOf.size()) return fail("bad dim reference in op");
        op.dims.push_back(dimOf[j]);
      }
      for (uint64_t k = 0, ni = r.count(); k < ni && r.ok(); ++k) op.ints.push_back(r.s());
      for (uint64_t k = 0, ns = r.count(); k < ns && r.ok(); ++k) {
        const uint64_t s = r.u();
        if (s >= symOf.size()) return fail("bad symbol reference");
        op.symbols.push_back(symOf[s]);
      }
      reg->ops.push_back(std::move(op));
    }
  }
  if (!r.ok()) return fail("corrupt metadata");
  auto badIds = [&](const std::vector<ValueId>& vs) {
    return std::any_of(vs.begin(), vs.end(), [&](ValueId v) { return v >= m->numValues(); });
  };
  for (const Region* reg : {&m->init, &m->exec}) {
    if (badIds(reg->args) || badIds(reg->state)) return fail("bad value reference");
    for (const Op& op : reg->ops)
      if (badIds(op.operands) || badIds(op.outs) || badIds(op.results)) return fail("bad value reference");
  }
  st = Status();
  return m;
}

Status writeLkmFile(const Model& m, const std::string& path) {
  Status st;
  std::vector<uint8_t> bytes = writeLkm(m, st);
  if (!st) return st;
  std::FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) return Status::error("cannot open " + path + " for writing");
  const size_t n = std::fwrite(bytes.data(), 1, bytes.size(), f);
  const bool closed = std::fclose(f) == 0;
  if (n != bytes.size() || !closed) return Status::error("failed writing " + path);
  return Status();
}

std::unique_ptr<Model> readLkmFile(const std::string& path, Status& st) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) {
    st = Status::error("cannot open " + path);
    return nullptr;
  }
  struct stat sb;
  if (::fstat(fd, &sb) != 0 || sb.st_size <= 0) {
    ::close(fd);
    st = Status::error(sb.st_size <= 0 ? "lkm: file too small" : "cannot stat " + path);
    return nullptr;
  }
  const size_t size = static_cast<size_t>(sb.st_size);
  void* p = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (p == MAP_FAILED) {
    st = Status::error("cannot mmap " + path);
    return nullptr;
  }
  std::shared_ptr<const void> owner(p, [size](const void* q) { ::munmap(const_cast<void*>(q), size); });
  return readLkm(static_cast<const uint8_t*>(p), size, owner, st);
}

}  // namespace lkrt

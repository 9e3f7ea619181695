// TEST INFRASTRUCTURE ONLY. A driver over the reference's own IR library (lariaus/lokinfer src/ir, src/compiler,
// compiled from /root/reference by oracle/ref_ir.mk into oracle/_ref/lkm-ref-tool), used in the build container
// to write the golden text-IR and .lkm fixtures under tests/golden/ir/ (tests/golden/make_ir_golden.py).
//
//   lkm-ref-tool print    IN.lkir                 parse, verify, print
//   lkm-ref-tool passes   LIST IN.lkir            parse, verify, run the comma-separated passes, print
//   lkm-ref-tool to-lkm   LIST IN.lkir OUT.lkm    as `passes` (LIST may be "-": none), then give every internal
//                                                 constant deterministic bytes (fixture_bytes below) and write
//   lkm-ref-tool from-lkm IN.lkm                  read, verify, print
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "lokinfer/compiler/passes.h"
#include "lokinfer/ir/binary.h"
#include "lokinfer/ir/text.h"
#include "lokinfer/ir/verify.h"

namespace {

int die(const std::string& msg) {
  std::fprintf(stderr, "error: %s\n", msg.c_str());
  return 1;
}

// Byte k of constant `name`: (k * 29 + sum of the name's bytes) mod 251 (the same rule as the Python test).
std::shared_ptr<std::vector<uint8_t>> fixtureBytes(const std::string& name, size_t n) {
  unsigned s = 0;
  for (unsigned char c : name) s += c;
  auto v = std::make_shared<std::vector<uint8_t>>(n);
  for (size_t k = 0; k < n; ++k) (*v)[k] = static_cast<uint8_t>((k * 29 + s) % 251);
  return v;
}

std::vector<std::string> split(const std::string& s) {
  std::vector<std::string> out;
  if (s == "-") return out;
  std::stringstream ss(s);
  std::string p;
  while (std::getline(ss, p, ',')) out.push_back(p == "pipeline" ? "" : p);
  if (out.size() == 1 && out[0].empty()) return lk::defaultPipeline();
  return out;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 3) return die("usage: lkm-ref-tool print|passes|to-lkm|from-lkm ...");
  const std::string mode = argv[1];
  if (mode == "from-lkm") {
    auto m = lk::readModelFile(argv[2]);
    if (!m) return die(m.status().message());
    if (auto s = lk::verifyModel(**m); !s) return die(s.message());
    std::fputs(lk::printModel(**m).c_str(), stdout);
    return 0;
  }
  const char* in = mode == "print" ? argv[2] : argc > 3 ? argv[3] : nullptr;
  if (!in) return die("missing input");
  std::ifstream f(in);
  if (!f) return die(std::string("cannot open ") + in);
  std::stringstream buf;
  buf << f.rdbuf();
  auto m = lk::parseModel(buf.str());
  if (!m) return die(m.status().message());
  if (auto s = lk::verifyModel(**m); !s) return die(s.message());
  if (mode != "print") {
    std::vector<std::string> passes = split(argv[2]);
    if (auto s = lk::runPasses(**m, passes, true); !s) return die(s.message());
  }
  if (mode == "to-lkm") {
    if (argc < 5) return die("missing output");
    for (auto& c : (*m)->constants) {
      size_t n = lk::dtypeSize(c.type->dtype);
      for (auto d : c.type->shape) n *= static_cast<size_t>(d->value);
      auto bytes = fixtureBytes(c.name, n);
      c.bytes = bytes->data();
      c.size = n;
      c.owner = bytes;
    }
    if (auto s = lk::writeModelFile(**m, argv[4]); !s) return die(s.message());
    return 0;
  }
  std::fputs(lk::printModel(**m).c_str(), stdout);
  return 0;
}

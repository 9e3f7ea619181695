# Builds the reference's portable IR + compiler sources (lariaus/lokinfer src/ir, src/compiler, tools/lokinfer_opt.cpp)
# straight from /root/reference into oracle/_ref/ with g++, plus oracle/lkm_ref_tool.cpp (this repo's driver for
# writeModelFile / readModelFile). TEST INFRASTRUCTURE ONLY: used in the build container to write the golden text-IR
# and .lkm fixtures under tests/golden/ (tests/golden/make_ir_golden.py); nothing in the product links it.
#   make -f oracle/ref_ir.mk            (from the repo root)
REF ?= /root/reference
OUT = oracle/_ref
CXX ?= g++
CXXFLAGS = -O1 -std=c++20 -I$(REF)/include -I$(REF)/src/compiler -w
IR_SRCS = $(wildcard $(REF)/src/ir/*.cpp) $(wildcard $(REF)/src/compiler/*.cpp)

all: $(OUT)/lokinfer-opt $(OUT)/lkm-ref-tool

$(OUT)/lokinfer-opt: $(IR_SRCS) $(REF)/tools/lokinfer_opt.cpp
	mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -o $@ $^

$(OUT)/lkm-ref-tool: $(IR_SRCS) oracle/lkm_ref_tool.cpp
	mkdir -p $(OUT)
	$(CXX) $(CXXFLAGS) -o $@ $^

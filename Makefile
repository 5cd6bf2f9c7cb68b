# Build of the MI355X (gfx950) tinytorch backend.
#
#   make lib      -> build/libtinytorch.so          (C ABI: tensor.h, autograd.h, tt_hip.h)
#   make pybind   -> build/tinytorch_pybind<EXT>    (Node API, links libtinytorch.so)
#   make oracle   -> oracle/build/liborc.so          (CPU restatement, test-only)
#   make ref      -> oracle/_ref/libtinytorch_ref.so (reference sources, when present)
# Target names and artefact names follow the reference Makefile:11-22.
ROCM    ?= /opt/rocm
HIPCC   ?= $(ROCM)/bin/hipcc
CC      ?= gcc
CXX     ?= g++
ARCH    ?= gfx950
BUILD   := build
CSRC    := tinytorch_amd/csrc

# -packed-fp32-ops off: the compiler generates no packed fp32 instructions
# (v_pk_*_f32); some of their forms have given wrong results on this hardware
HIPFLAGS := --offload-arch=$(ARCH) -O3 -fPIC -std=c++17 -Iinclude -I$(CSRC) \
            -Xclang -target-feature -Xclang -packed-fp32-ops -Wno-unused-command-line-argument
CFLAGS_HOST := -O2 -fPIC -std=c11 -Wall -Wextra -D__HIP_PLATFORM_AMD__ -I$(ROCM)/include \
               -Iinclude -I$(CSRC)

HOST_SRCS := $(CSRC)/runtime.c $(CSRC)/tensor.c $(CSRC)/ops.c $(CSRC)/autograd.c $(CSRC)/dataset.c
HIP_SRCS  := $(CSRC)/gemm.hip $(CSRC)/conv.hip $(CSRC)/elementwise.hip $(CSRC)/spatial.hip \
             $(CSRC)/head.hip
HDRS      := $(wildcard include/*.h) $(wildcard $(CSRC)/*.h)
HOST_OBJS := $(patsubst $(CSRC)/%.c,$(BUILD)/obj/%.o,$(HOST_SRCS))
HIP_OBJS  := $(patsubst $(CSRC)/%.hip,$(BUILD)/obj/%.o,$(HIP_SRCS))

PYBIND_INC := $(shell python3 -m pybind11 --includes 2>/dev/null)
EXT_SUFFIX := $(shell python3-config --extension-suffix 2>/dev/null || echo ".so")

all: lib pybind

$(BUILD)/obj/%.o: $(CSRC)/%.c $(HDRS) | $(BUILD)/obj
	$(CC) $(CFLAGS_HOST) -c $< -o $@

# the GEMM may fuse multiply-adds (it is tolerance-checked); the bandwidth
# kernels are compiled without contraction so their sums round like the
# reference's separate multiply and add
$(BUILD)/obj/gemm.o: $(CSRC)/gemm.hip $(HDRS) | $(BUILD)/obj
	$(HIPCC) $(HIPFLAGS) -c $< -o $@

# direct convolution: MFMA accumulators in VGPRs (the AGPR form made the
# compiler copy accumulators between register files every loop iteration)
$(BUILD)/obj/conv.o: $(CSRC)/conv.hip $(HDRS) | $(BUILD)/obj
	$(HIPCC) $(HIPFLAGS) -ffp-contract=off -mllvm -amdgpu-mfma-vgpr-form=1 -c $< -o $@

$(BUILD)/obj/%.o: $(CSRC)/%.hip $(HDRS) | $(BUILD)/obj
	$(HIPCC) $(HIPFLAGS) -ffp-contract=off -c $< -o $@

$(BUILD)/libtinytorch.so: $(HOST_OBJS) $(HIP_OBJS)
	$(HIPCC) --offload-arch=$(ARCH) -shared -fPIC -o $@ $^ -Wl,-Bsymbolic -Wl,-soname,libtinytorch.so -lz

$(BUILD)/tinytorch_pybind$(EXT_SUFFIX): $(CSRC)/bindings.cpp $(BUILD)/libtinytorch.so $(HDRS)
	$(CXX) -O2 -fPIC -shared -std=c++17 $(PYBIND_INC) -Iinclude -o $@ $< \
	    -L$(BUILD) -ltinytorch -Wl,-rpath,'$$ORIGIN'

$(BUILD)/obj:
	mkdir -p $@

lib: $(BUILD)/libtinytorch.so

# the library with phase timestamps compiled in (TT_PHASE_PROBE, probe.h) for
# `bench.py --phases`; a separate build tree, never loaded by the tests
probe:
	$(MAKE) BUILD=$(BUILD)/probe HIPFLAGS="$(HIPFLAGS) -DTT_PHASE_PROBE" lib
pybind: $(BUILD)/tinytorch_pybind$(EXT_SUFFIX)

oracle:
	$(MAKE) -C oracle

ref:
	$(MAKE) -C oracle ref

clean:
	rm -rf $(BUILD)

.PHONY: all lib pybind oracle ref clean probe

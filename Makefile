# Build of the MI355X decode megakernel.
#   make lib    -> megakernel_amd/megakernel.so   (the reference's `make lib` target)
#   make trace-lib -> megakernel_amd/megakernel_trace.so (trace events compiled in)
#   make clean
# Code objects are built for gfx950 only.  Packed-FP32 instructions are turned
# off for every HIP translation unit (they are not used by hand either).
# Translation units compile to objects under _build/ (make -j builds them in
# parallel) and link into one shared library.

HIPCC      ?= /opt/rocm/bin/hipcc
ARCH       ?= gfx950
HIPFLAGS   := --offload-arch=$(ARCH) -O3 -std=c++17 -fPIC \
              -Xclang -target-feature -Xclang -packed-fp32-ops \
              -Wno-unused-command-line-argument
CSRC       := megakernel_amd/csrc
LIB        := megakernel_amd/megakernel.so
SRCS       := $(CSRC)/megakernel.hip $(CSRC)/decode_baseline.hip $(CSRC)/decode_qwen3.hip \
              $(CSRC)/decode_tiny.hip $(CSRC)/batch.hip $(CSRC)/ops.hip $(CSRC)/selftest.hip
OBJS       := $(patsubst $(CSRC)/%.hip,_build/%.o,$(SRCS))
HDRS       := $(wildcard $(CSRC)/*.h) include/megakernel.h

# Library with the poll-level trace events compiled in (bench.py --trace
# prints the hand-off decomposition from it; investigation only).
TRACE_LIB  := megakernel_amd/megakernel_trace.so
TRACE_OBJS := $(patsubst $(CSRC)/%.hip,_build/trace/%.o,$(SRCS))

.PHONY: all lib trace-lib clean asm

all: lib

lib: $(LIB)

_build/%.o: $(CSRC)/%.hip $(HDRS)
	@mkdir -p _build
	$(HIPCC) $(HIPFLAGS) -Iinclude -c $< -o $@

$(LIB): $(OBJS)
	$(HIPCC) $(HIPFLAGS) -shared $(OBJS) -o $@.tmp
	mv $@.tmp $@

_build/trace/%.o: $(CSRC)/%.hip $(HDRS)
	@mkdir -p _build/trace
	$(HIPCC) $(HIPFLAGS) -DMK_TRACE_EVENTS=1 -Iinclude -c $< -o $@

trace-lib: $(TRACE_LIB)

$(TRACE_LIB): $(TRACE_OBJS)
	$(HIPCC) $(HIPFLAGS) -shared $(TRACE_OBJS) -o $@.tmp
	mv $@.tmp $@

# Device assembly for inspection (not part of the product).
asm: $(SRCS) $(HDRS)
	@mkdir -p _build
	$(HIPCC) $(HIPFLAGS) -Iinclude --cuda-device-only -S $(CSRC)/megakernel.hip -o _build/megakernel-gfx950.s

clean:
	rm -f $(LIB) $(LIB).tmp $(OBJS) $(TRACE_LIB) $(TRACE_OBJS)

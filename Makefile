# Build of the MI355X decode megakernel.
#   make lib    -> megakernel_amd/megakernel.so   (the reference's `make lib` target)
#   make clean
# Code objects are built for gfx950 only.  Packed-FP32 instructions are turned
# off for every HIP translation unit (they are not used by hand either).

HIPCC      ?= /opt/rocm/bin/hipcc
ARCH       ?= gfx950
HIPFLAGS   := --offload-arch=$(ARCH) -O3 -std=c++17 -fPIC \
              -Xclang -target-feature -Xclang -packed-fp32-ops \
              -Wno-unused-command-line-argument
CSRC       := megakernel_amd/csrc
LIB        := megakernel_amd/megakernel.so
SRCS       := $(CSRC)/megakernel.hip $(CSRC)/batch.hip $(CSRC)/ops.hip $(CSRC)/selftest.hip
HDRS       := $(wildcard $(CSRC)/*.h) include/megakernel.h

.PHONY: all lib clean asm

all: lib

lib: $(LIB)

$(LIB): $(SRCS) $(HDRS)
	$(HIPCC) $(HIPFLAGS) -shared -Iinclude $(SRCS) -o $@.tmp
	mv $@.tmp $@

# Device assembly for inspection (not part of the product).
asm: $(SRCS) $(HDRS)
	$(HIPCC) $(HIPFLAGS) -Iinclude --cuda-device-only -S $(SRCS) -o _build/megakernel-gfx950.s

clean:
	rm -f $(LIB) $(LIB).tmp

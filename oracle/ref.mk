# Builds the reference's own kernels for the oracle checks (TEST ONLY):
#   _ref/sam3_kernels.gfx950.co  /root/reference/sam3_kernels.cl compiled
#                                unchanged by ROCm clang for gfx950, with the
#                                reference's build options (-cl-std=CL1.2
#                                -cl-mad-enable, ocl_backend.c:167-170)
#   _ref/libsam3ref.so           ref_harness.c: launches those kernels through
#                                the OpenCL runtime like the reference host
# Outputs go to _ref/ only (git-ignored); nothing is copied from the reference.
REF ?= /root/reference
ROCM ?= /opt/rocm
CLANG = $(ROCM)/lib/llvm/bin/clang

all: _ref/sam3_kernels.gfx950.co _ref/libsam3ref.so

_ref/sam3_kernels.gfx950.co: $(REF)/sam3_kernels.cl
	mkdir -p _ref
	$(CLANG) -x cl -cl-std=CL1.2 -cl-mad-enable -Xclang -finclude-default-header \
	    -target amdgcn-amd-amdhsa -mcpu=gfx950 -O3 -Wno-everything -o $@ $<

_ref/libsam3ref.so: ref_harness.c
	mkdir -p _ref
	gcc -O2 -fPIC -shared -std=gnu11 -Wall -I$(ROCM)/include -o $@ $< -lOpenCL -lm

clean:
	rm -rf _ref

.PHONY: all clean

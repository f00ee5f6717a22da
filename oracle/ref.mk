# oracle/ref.mk -- compile the reference's own CPU GEMM / int4-quant translation units IN PLACE from
# the read-only reference tree and link them, with this directory's driver, into _ref/libork_ref.so.
# Nothing is copied from the reference; objects and the library go to _ref/ (git-ignored; it travels
# to the GPU box as a built artefact). clang is used because the reference headers need _Float16,
# which gcc-11 rejects on x86. Flags follow the reference Makefile (-O2), plus section splitting so
# the linker can drop every function the driver does not reach; -z defs proves nothing is left
# unresolved (no stand-in symbols are supplied).
REF     ?= /root/reference
HERE    := $(dir $(abspath $(lastword $(MAKEFILE_LIST))))
OUT     := $(HERE)_ref
CLANG   ?= /opt/rocm/llvm/bin/clang
CFLAGS  := -O2 -fPIC -std=gnu11 -w -ffp-contract=off -ffunction-sections -fdata-sections \
           -I$(REF)/include -I$(REF)/src -pthread
SRCS    := $(REF)/src/npu/core/buf.c $(REF)/src/npu/i4/quant.c
OBJS    := $(OUT)/buf.o $(OUT)/quant.o $(OUT)/ref_driver.o

$(OUT)/libork_ref.so: $(OBJS)
	echo '{ global: ref_*; local: *; };' > $(OUT)/ref.map
	$(CLANG) -shared -fuse-ld=lld -Wl,--gc-sections -Wl,--version-script=$(OUT)/ref.map -Wl,-z,defs \
	    -o $@ $(OBJS) -lm -pthread

$(OUT)/buf.o: $(REF)/src/npu/core/buf.c
	mkdir -p $(OUT)
	$(CLANG) $(CFLAGS) -c $< -o $@
$(OUT)/quant.o: $(REF)/src/npu/i4/quant.c
	mkdir -p $(OUT)
	$(CLANG) $(CFLAGS) -c $< -o $@
$(OUT)/ref_driver.o: $(HERE)ref_driver.c
	mkdir -p $(OUT)
	$(CLANG) $(CFLAGS) -c $< -o $@

# The same translation units with -fopenmp: the reference's `#pragma omp parallel for ... if(M>1)` over rows
# (src/npu/core/buf.c:438) becomes live, as in the reference Makefile's OpenMP tool targets (:192). This is the
# all-cores CPU baseline; libomp comes from the ROCm LLVM tree (rpath below).
OMPLIB  := /opt/rocm/llvm/lib
OMPOBJS := $(OUT)/omp/buf.o $(OUT)/omp/quant.o $(OUT)/omp/ref_driver.o
$(OUT)/libork_ref_omp.so: $(OMPOBJS)
	echo '{ global: ref_*; local: *; };' > $(OUT)/ref.map
	$(CLANG) -shared -fuse-ld=lld -fopenmp -Wl,--gc-sections -Wl,--version-script=$(OUT)/ref.map -Wl,-z,defs \
	    -L$(OMPLIB) -Wl,-rpath,$(OMPLIB) -o $@ $(OMPOBJS) -lm -pthread
$(OUT)/omp/buf.o: $(REF)/src/npu/core/buf.c
	mkdir -p $(OUT)/omp
	$(CLANG) $(CFLAGS) -fopenmp -c $< -o $@
$(OUT)/omp/quant.o: $(REF)/src/npu/i4/quant.c
	mkdir -p $(OUT)/omp
	$(CLANG) $(CFLAGS) -fopenmp -c $< -o $@
$(OUT)/omp/ref_driver.o: $(HERE)ref_driver.c
	mkdir -p $(OUT)/omp
	$(CLANG) $(CFLAGS) -fopenmp -c $< -o $@

# The reference's own example / test programs, compiled UNMODIFIED from the reference tree against this
# repository's drop-in headers (include/ork_npu.h) and linked to libork_npu.so: C consumers of the reference API
# running on the MI355X engine, each checked by its own embedded goldens and assertions (tests/test_gpu_dropin.py
# runs the device ones on the GPU, tests/test_host.py the offline one here).
ROOT    := $(abspath $(HERE)..)
EXAMPLES := quant test_matmul i4 test_sn3 test_grouped_i8 test_i4_dump_cpu test_pack_gate test_offline_load
DROPINS := $(addprefix $(OUT)/,$(addsuffix _on_mi355x,$(EXAMPLES)))
$(OUT)/%_on_mi355x: $(REF)/examples/%.c $(ROOT)/ork-driver_amd/libork_npu.so $(wildcard $(ROOT)/include/*.h $(ROOT)/include/ork/*.h)
	mkdir -p $(OUT)
	$(CLANG) -O2 -std=gnu11 -w -I$(ROOT)/include $< -o $@ -L$(ROOT)/ork-driver_amd -lork_npu \
	    -Wl,-rpath,'$$ORIGIN/../../ork-driver_amd' -lm

dropin: $(DROPINS)
.PHONY: dropin

# Builds the reference's own C++ sources for this path, straight from the
# read-only reference tree, into oracle/_ref/ (git-ignored and kept out of the
# snapshots that GPU runs receive: only the CPU test suite uses them, and no
# reference code runs beside the GPU).  Nothing here is copied into the
# repository.
#
#   make -f oracle/ref.mk            (REF defaults to /root/reference)
#
# libkvsnap_io_ref.so           csrc/dataplane/io.cpp: CRC32C + pread/pwrite pool
#                               (libc + <nmmintrin.h> only, as the reference's own
#                               tests/unit/test_native_io.py:33-37 compiles it)
# libkvsnap_pool_fakecuda_ref.so csrc/dataplane/cuda_pool.cpp against the reference's
#                               own CPU test runtime tests/native/fake_cuda.cpp
#                               (test_independent_native.py:24-26): a control-flow
#                               oracle for the pinned pool, never a data oracle.
REF ?= /root/reference
OUT := $(patsubst %/,%,$(dir $(lastword $(MAKEFILE_LIST))))/_ref

all: $(OUT)/libkvsnap_io_ref.so $(OUT)/libkvsnap_pool_fakecuda_ref.so

$(OUT)/libkvsnap_io_ref.so: $(REF)/csrc/dataplane/io.cpp
	mkdir -p $(OUT)
	g++ -std=c++17 -O2 -shared -fPIC -pthread -Wall -Wextra -o $@ $<

$(OUT)/libkvsnap_pool_fakecuda_ref.so: $(REF)/csrc/dataplane/cuda_pool.cpp $(REF)/tests/native/fake_cuda.cpp
	mkdir -p $(OUT)
	g++ -std=c++17 -O2 -shared -fPIC -pthread -Wl,-Bsymbolic -I$(REF)/tests/native -o $@ $^

.PHONY: all

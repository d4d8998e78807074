# Builds the reference's own CPU sources, where they lie, into oracle/_ref/libref.so.
#
# Test infrastructure only: the library is the second checker of the C oracle (oracle.c) and the
# optional "reference" CPU baseline of bench.py. Nothing here is copied into the repository; the
# sources are read from REF (the read-only reference tree) and only the built .so is written.
#
#   make -f oracle/ref.mk            (from the repository root)
#
# Sources (all plain C++17, no HIP, no ggml):
#   src/quant_types.cpp   GGUF block decoders (qt_*)
#   src/quantize.cpp      weight encoders (qz_*); needs -ffp-contract=off (it #errors under fast math)
#   src/quantize_iq.cpp   IQ encoders, referenced by quantize.cpp's row driver
#   src/expert_cpu.cpp    CPU expert matvecs (scalar + AVX-512 VNNI, chosen at run time)
#   src/gguf_mmap.cpp     the GGUF reader (gguf_*)

REF ?= /root/reference
ORACLE_DIR := $(dir $(lastword $(MAKEFILE_LIST)))
OUT := $(ORACLE_DIR)_ref
SRCS := $(REF)/src/quant_types.cpp $(REF)/src/quantize.cpp $(REF)/src/quantize_iq.cpp $(REF)/src/expert_cpu.cpp \
        $(REF)/src/gguf_mmap.cpp
CXXFLAGS := -std=c++17 -O2 -fPIC -ffp-contract=off -fno-fast-math -I$(REF)/src -w

$(OUT)/libref.so: $(SRCS) $(lastword $(MAKEFILE_LIST))
	@mkdir -p $(OUT)
	g++ $(CXXFLAGS) -shared -o $@ $(SRCS) -lpthread

.PHONY: clean
clean:
	rm -rf $(OUT)

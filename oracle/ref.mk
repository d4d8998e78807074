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
# plus this directory's ref_bench.cpp (a timing harness of our own around the reference's CPU matvecs).

REF ?= /root/reference
ORACLE_DIR := $(dir $(lastword $(MAKEFILE_LIST)))
OUT := $(ORACLE_DIR)_ref
# the encoders need -ffp-contract=off (the reference's Makefile:299-300; quantize.cpp #errors under fast math);
# the CPU matvecs are built as the reference builds expert_cpu.cpp (Makefile:387: -O3, default contraction)
SRCS := $(REF)/src/quant_types.cpp $(REF)/src/quantize.cpp $(REF)/src/quantize_iq.cpp $(REF)/src/gguf_mmap.cpp
FAST_SRCS := $(REF)/src/expert_cpu.cpp $(ORACLE_DIR)ref_bench.cpp
CXXFLAGS := -std=c++17 -O2 -fPIC -ffp-contract=off -fno-fast-math -I$(REF)/src -w
FASTFLAGS := -std=c++17 -O3 -fPIC -I$(REF)/src -w

$(OUT)/libref.so: $(SRCS) $(FAST_SRCS) $(lastword $(MAKEFILE_LIST))
	@mkdir -p $(OUT)
	g++ $(FASTFLAGS) -c $(REF)/src/expert_cpu.cpp -o $(OUT)/expert_cpu.o
	g++ $(FASTFLAGS) -c $(ORACLE_DIR)ref_bench.cpp -o $(OUT)/ref_bench.o
	g++ $(CXXFLAGS) -shared -o $@ $(SRCS) $(OUT)/expert_cpu.o $(OUT)/ref_bench.o -lpthread

.PHONY: clean
clean:
	rm -rf $(OUT)

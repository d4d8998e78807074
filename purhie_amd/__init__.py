"""MI355X-native quantized-weight matrix products (GGUF Q8_0 / Q4_K / Q6_K / ROCmFP4) behind the
reference's qmatvec / quant_types C ABI. The compute lives in libpurhie_qmv.so (HIP, gfx950);
purhie_amd.qmatvec is its ctypes mirror."""

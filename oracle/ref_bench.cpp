// ref_bench.cpp -- timing harness around the reference's own CPU matvecs (src/expert_cpu.cpp), linked into
// oracle/_ref/libref.so by oracle/ref.mk. Test infrastructure: bench.py's cpu_baseline leg only.
//
// Times `reps` passes of y = W x over rotating copies of W (copy c at W + c * N * rb), each pass splitting the
// N rows into chunks of `chunk` rows that the reference's cpu_matvec_q8_q8 (Q8_0) or cpu_matvec_fp4fast_q8
// (ROCmFP4_FAST) computes; the reference picks its AVX-512 VNNI or scalar body at run time (have_vnni,
// src/expert_cpu.cpp:33-37). threads > 0: that many persistent threads (the caller one of them) take each pass's
// chunks from a shared counter and meet at a barrier after it (all cores);
// threads <= 0: the reference's own pool (cpu_parallel_for, src/expert_cpu.cpp:266-333: the cores less one, at
// most 15 workers, plus the caller).
#include <atomic>
#include <chrono>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <functional>
#include <thread>
#include <vector>

void cpu_matvec_q8_q8(const void *W, size_t row_bytes, int N, int K, const int8_t *q, const float *d, float *y);
void cpu_matvec_fp4fast_q8(const void *W, size_t row_bytes, int N, int K, const int8_t *q, const float *d, float *y);
void cpu_parallel_for(int n, const std::function<void(int)> &fn);

extern "C" {

// the reference's own test for its VNNI body (src/expert_cpu.cpp:33-37)
int refb_have_vnni(void) {
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni") && !getenv("INFERENCE_CPU_SCALAR");
}

double refb_matvec(int type, const uint8_t *W, size_t rb, int N, int K, int copies, const int8_t *q, const float *d,
                   float *y, int threads, int reps, int chunk) {
    auto mv = type == 8 ? cpu_matvec_q8_q8 : cpu_matvec_fp4fast_q8;
    const int nchunk = (N + chunk - 1) / chunk;
    auto item = [&](int r, int i) {
        const uint8_t *Wc = W + (size_t)(r % copies) * (size_t)N * rb;
        const int r0 = i * chunk, n = N - r0 < chunk ? N - r0 : chunk;
        mv(Wc + (size_t)r0 * rb, rb, n, K, q, d, y + r0);
    };
    if (threads <= 0) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int r = 0; r < reps; ++r) cpu_parallel_for(nchunk, [&](int i) { item(r, i); });
        return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    }
    // persistent threads; pass r hands out its chunks from next[r & 1] and ends at a spin barrier (the last thread
    // to arrive resets the other counter for pass r + 1, then releases the others)
    std::atomic<int> next[2], arrived{0}, phase{0};
    next[0] = 0;
    next[1] = 0;
    auto barrier = [&](int r) {
        const int ph = phase.load(std::memory_order_acquire);
        if (arrived.fetch_add(1, std::memory_order_acq_rel) + 1 == threads) {
            arrived.store(0, std::memory_order_relaxed);
            next[(r + 1) & 1].store(0, std::memory_order_relaxed);
            phase.fetch_add(1, std::memory_order_acq_rel);
        } else {
            while (phase.load(std::memory_order_acquire) == ph) __builtin_ia32_pause();
        }
    };
    std::chrono::steady_clock::time_point t0, t1;
    auto body = [&](int k) {
        barrier(-1);  // (every thread started; pass 0 uses next[0], reset above)
        if (k == 0) t0 = std::chrono::steady_clock::now();
        for (int r = 0; r < reps; ++r) {
            for (int i; (i = next[r & 1].fetch_add(1)) < nchunk;) item(r, i);
            barrier(r);
        }
        if (k == 0) t1 = std::chrono::steady_clock::now();
    };
    std::vector<std::thread> th;
    th.reserve((size_t)threads);
    for (int k = 1; k < threads; ++k) th.emplace_back(body, k);
    body(0);
    for (auto &t : th) t.join();
    return std::chrono::duration<double>(t1 - t0).count();
}

}  // extern "C"

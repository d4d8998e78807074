// out_scale.cpp -- the output-scale registry behind qmatvec_set_out_scale / qmatvec_drop_out_scales
// (reference interface: src/qmatvec.h:21-26; semantics of src/qmatvec.cpp:175-253).
//
// Design: launches only read the registry, and registrations are rare (once per model load). So the registry is
// an immutable table, replaced as a whole on every change and published through an atomic shared pointer:
//   * a lookup takes no lock. It loads the current table and binary-searches its ranges (sorted by start
//     address) for the one holding W;
//   * a change (under a writer mutex) copies the table, edits the copy, and publishes it. A launch still
//     holding the old table keeps it alive until its lookup ends.
// Overlapping registrations resolve as the reference's do: the earliest registration that holds W wins. Each
// range keeps its registration number; `reach` (the largest end address among ranges that start at or before a
// range) bounds the backward scan from the last range that starts at or before W.
#include "out_scale.h"

#include <algorithm>
#include <memory>
#include <mutex>
#include <vector>

namespace pq {
namespace {

struct Range {
    const char *lo, *hi;  // the matrix's bytes
    const float *s;       // n factors: the matrix's (n = 1) or one per stacked expert
    int n;
    const void *owner;
    unsigned long long seq;  // registration order
};

struct Table {
    std::vector<Range> r;            // sorted by lo
    std::vector<const char *> reach; // reach[i] = max(r[0..i].hi)
};

std::shared_ptr<const Table> g_table;  // (read and replaced with the atomic shared_ptr free functions)
std::mutex g_write;
unsigned long long g_seq = 0;

void publish(std::vector<Range> v) {
    auto t = std::make_shared<Table>();
    std::sort(v.begin(), v.end(), [](const Range &a, const Range &b) { return a.lo < b.lo || (a.lo == b.lo && a.seq < b.seq); });
    t->reach.resize(v.size());
    const char *m = nullptr;
    for (size_t i = 0; i < v.size(); ++i) {
        m = i == 0 || v[i].hi > m ? v[i].hi : m;
        t->reach[i] = m;
    }
    t->r = std::move(v);
    std::atomic_store(&g_table, std::shared_ptr<const Table>(std::move(t)));
}

std::vector<Range> current() {
    const std::shared_ptr<const Table> t = std::atomic_load(&g_table);
    return t ? t->r : std::vector<Range>();
}

}  // namespace

bool scale_find(const void *W, ScaleHit &h) {
    if (!W) return false;
    const std::shared_ptr<const Table> t = std::atomic_load(&g_table);
    if (!t || t->r.empty()) return false;
    const char *w = (const char *)W;
    // ranges starting at or before w: [0, i)
    size_t i = (size_t)(std::upper_bound(t->r.begin(), t->r.end(), w, [](const char *x, const Range &a) { return x < a.lo; }) -
                        t->r.begin());
    const Range *best = nullptr;
    while (i-- > 0 && t->reach[i] > w) {
        const Range &a = t->r[i];
        if (w < a.hi && (!best || a.seq < best->seq)) best = &a;
    }
    if (!best) return false;
    h.s = best->s;
    h.n = best->n;
    h.lo = best->lo;
    h.hi = best->hi;
    return true;
}

float scale_dense(const void *W) {
    ScaleHit h;
    if (!scale_find(W, h)) return 1.0f;
    if (h.n == 1) return h.s[0];
    const size_t per = (size_t)(h.hi - h.lo) / (size_t)h.n;
    return h.s[(size_t)((const char *)W - h.lo) / per];
}

}  // namespace pq

extern "C" {

int qmatvec_set_out_scale(const void *owner, const void *W, size_t bytes, const float *s, int n) {
    if (!W || !s || n < 1 || bytes % (size_t)n != 0) return -1;
    std::lock_guard<std::mutex> lk(pq::g_write);
    std::vector<pq::Range> v = pq::current();
    v.push_back({(const char *)W, (const char *)W + bytes, s, n, owner, pq::g_seq++});
    pq::publish(std::move(v));
    return 0;
}

void qmatvec_drop_out_scales(const void *owner) {
    std::lock_guard<std::mutex> lk(pq::g_write);
    std::vector<pq::Range> v = pq::current();
    const size_t before = v.size();
    v.erase(std::remove_if(v.begin(), v.end(), [owner](const pq::Range &a) { return a.owner == owner; }), v.end());
    if (v.size() != before) pq::publish(std::move(v));
}

}  // extern "C"

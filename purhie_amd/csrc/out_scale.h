// out_scale.h -- lookups into the output-scale registry (out_scale.cpp), for the launch code of qmatvec.cpp.
#pragma once

#include "../../include/qmatvec.h"

namespace pq {

// the registration holding the matrix pointer W: its n factors s (caller memory, readable by the CPU and the GPU)
// and its byte range
struct ScaleHit {
    const float *s;
    int n;
    const char *lo, *hi;
};
bool scale_find(const void *W, ScaleHit &h);

// the factor of a launch on rows from W: 1 when nothing is registered, the matrix's s[0], or, for W inside n
// stacked experts, the factor of the expert W points into (read on the host)
float scale_dense(const void *W);

}  // namespace pq

// SoftmaxCPU: host (CPU execution provider) softmax of the "xmetai_plugins"
// domain.  Reference: csrc/softmax_cpu/softmax_cpu_ort.cpp:20-114.
//
// For every line of the tensor along `axis`: m = max_a x[a]; e[a] =
// exp(x[a] - m); s = e[0] + e[1] + ... in axis order (fp32); y[a] = e[a] *
// (s > 0 ? 1/s : 0).  The loops run with the lines that share an outer index
// side by side (the innermost loop walks the contiguous `inner` dimension),
// but every line sees exactly that sequence of fp32 operations, so the result
// is the same bit pattern as evaluating one line at a time.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

#include "xm_common.h"
#include "xmetai_recurrent.h"

namespace xm {
namespace {

void SoftmaxLines(const float *in, float *out, size_t outer, size_t axis_dim, size_t inner) {
    std::vector<float> mx(inner), sum(inner);
    for (size_t o = 0; o < outer; ++o) {
        const float *x = in + o * axis_dim * inner;
        float *y = out + o * axis_dim * inner;
        std::fill(mx.begin(), mx.end(), -std::numeric_limits<float>::infinity());
        for (size_t a = 0; a < axis_dim; ++a) {
            const float *xa = x + a * inner;
            for (size_t i = 0; i < inner; ++i) mx[i] = std::max(mx[i], xa[i]);
        }
        std::fill(sum.begin(), sum.end(), 0.0f);
        for (size_t a = 0; a < axis_dim; ++a) {
            const float *xa = x + a * inner;
            float *ya = y + a * inner;
            for (size_t i = 0; i < inner; ++i) {
                const float e = std::exp(xa[i] - mx[i]);
                ya[i] = e;
                sum[i] += e;
            }
        }
        for (size_t i = 0; i < inner; ++i) sum[i] = sum[i] > 0.0f ? 1.0f / sum[i] : 0.0f;   // inv_sum (:75)
        for (size_t a = 0; a < axis_dim; ++a) {
            float *ya = y + a * inner;
            for (size_t i = 0; i < inner; ++i) ya[i] *= sum[i];
        }
    }
}

}  // namespace
}  // namespace xm

extern "C" int xm_softmax_cpu(const float *in, const int64_t *shape, int32_t rank, int64_t axis, float *out,
                              char *errbuf, size_t errlen) {
    return xm::Guard(errbuf, errlen, [&] {
        if (rank < 0 || rank > XM_MAX_RANK || (rank > 0 && shape == nullptr))
            xm::Invalid("SoftmaxCPU input rank is out of range");
        size_t elements = 1;
        for (int32_t i = 0; i < rank; ++i) {
            if (shape[i] < 0) xm::Invalid("SoftmaxCPU input has a negative dimension");
            elements *= static_cast<size_t>(shape[i]);
        }
        if (elements == 0) return;   // reference :34-36: empty input, nothing to do (axis unchecked)
        if (in == nullptr || out == nullptr) xm::Invalid("SoftmaxCPU received a null tensor pointer");
        int64_t ax = axis;
        if (ax < 0) ax += rank;
        if (ax < 0 || ax >= rank) xm::Invalid("SoftmaxCPU axis out of range");   // reference :45
        size_t outer = 1, inner = 1;
        for (int64_t i = 0; i < ax; ++i) outer *= static_cast<size_t>(shape[i]);
        for (int64_t i = ax + 1; i < rank; ++i) inner *= static_cast<size_t>(shape[i]);
        xm::SoftmaxLines(in, out, outer, static_cast<size_t>(shape[ax]), inner);
    });
}

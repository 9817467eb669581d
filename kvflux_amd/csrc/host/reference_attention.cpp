// Host reference attention of the kvflux::v2 API (a CPU function of the API,
// not a path of the GPU operations). Same arithmetic as the reference's
// reference_attention (src/v2/reference_attention.cpp:28-91): inputs widened
// to double, dot products, the maximum-shifted exp and the normalisation in
// double, in the same loop order, output rounded to float -- so results are
// bit-identical to the reference's own CPU build.
#include "kvflux/v2/reference_attention.h"

#include <cmath>
#include <limits>
#include <stdexcept>

namespace kvflux::v2 {
namespace {

std::size_t product(std::size_t a, std::size_t b) {
    if (b != 0 && a > std::numeric_limits<std::size_t>::max() / b) {
        throw std::overflow_error("reference attention tensor size overflow");
    }
    return a * b;
}

void require_finite(const std::vector<float>& values) {
    for (const float x : values) {
        if (!std::isfinite(x)) throw std::invalid_argument("reference attention inputs must be finite");
    }
}

} // namespace

std::vector<float> reference_attention(const std::vector<float>& query, const std::vector<float>& key,
                                       const std::vector<float>& value, const AttentionShape& shape) {
    const std::size_t Tq = shape.query_tokens, Tk = shape.kv_tokens;
    const std::size_t Hq = shape.query_heads, H = shape.kv_heads, D = shape.head_size;
    if (Hq == 0 || H == 0 || D == 0 || Hq % H != 0 || Tq > Tk) {
        throw std::invalid_argument("invalid reference attention shape");
    }
    const std::size_t q_count = product(product(Tq, Hq), D);
    const std::size_t kv_count = product(product(Tk, H), D);
    if (query.size() != q_count || key.size() != kv_count || value.size() != kv_count) {
        throw std::invalid_argument("reference attention tensor size does not match shape");
    }
    require_finite(query);
    require_finite(key);
    require_finite(value);

    std::vector<float> out(q_count, 0.0f);
    if (Tq == 0) return out;
    const double scale = 1.0 / std::sqrt(static_cast<double>(D));
    const std::size_t group = Hq / H;
    std::vector<double> weight(Tk);
    for (std::size_t t = 0; t < Tq; ++t) {
        const std::size_t visible = Tk - Tq + t;  // last key position this query sees
        for (std::size_t qh = 0; qh < Hq; ++qh) {
            const std::size_t kvh = qh / group;
            const float* q = query.data() + (t * Hq + qh) * D;
            double top = -std::numeric_limits<double>::infinity();
            for (std::size_t j = 0; j <= visible; ++j) {
                const float* k = key.data() + (j * H + kvh) * D;
                double dot = 0.0;
                for (std::size_t d = 0; d < D; ++d) dot += static_cast<double>(q[d]) * k[d];
                weight[j] = dot * scale;
                if (weight[j] > top) top = weight[j];
            }
            double total = 0.0;
            for (std::size_t j = 0; j <= visible; ++j) {
                weight[j] = std::exp(weight[j] - top);
                total += weight[j];
            }
            float* o = out.data() + (t * Hq + qh) * D;
            for (std::size_t d = 0; d < D; ++d) {
                double acc = 0.0;
                for (std::size_t j = 0; j <= visible; ++j) {
                    acc += (weight[j] / total) * value[(j * H + kvh) * D + d];
                }
                o[d] = static_cast<float>(acc);
            }
        }
    }
    return out;
}

} // namespace kvflux::v2

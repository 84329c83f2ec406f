// extern "C" tsfm_timestral_encode_categorical (include/tsfm_attn.h): the categorical covariates of
// a Timestral forecast as numeric rows, on the host, before the forecast's device passes.
//
// Reference: src/timestral/forecaster.zig forecast (:86-103), encodingTarget (:201-217),
// encodeCategorical (:220-238), targetEncode (:243-289), slotOf (:292-301). The categories of a
// row are held sorted and deduplicated, and a code's category is found by binary search, so a row
// of len codes costs O(len log len).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

#include "../../include/tsfm_attn.h"
#include "abi_internal.hpp"

using tsfm::abi::fail;

namespace {

// Index of a finite code among the sorted categories, or -1 (NaN, infinities, unseen codes).
int64_t category_of(const std::vector<double>& cats, double code) {
    if (std::isnan(code)) return -1;
    const auto it = std::lower_bound(cats.begin(), cats.end(), code);
    return it != cats.end() && *it == code ? it - cats.begin() : -1;
}

// One code row of one series against its encoding target tg[0, t) (NaN outside the window).
void encode_row(const double* row, const double* tg, int64_t t, int64_t len, float* dst, std::vector<double>& cats,
                std::vector<double>& sums, std::vector<double>& counts) {
    double n_obs = 0.0, total = 0.0;
    for (int64_t i = 0; i < t; i++)
        if (std::isfinite(tg[i])) {
            n_obs += 1.0;
            total += tg[i];
        }
    const double mean = n_obs > 0.0 ? total / n_obs : 0.0;

    cats.clear();
    for (int64_t i = 0; i < t; i++)
        if (std::isfinite(row[i])) cats.push_back(row[i]);
    std::sort(cats.begin(), cats.end());
    cats.erase(std::unique(cats.begin(), cats.end()), cats.end());
    const int64_t missing = (int64_t)cats.size();  // the slot of NaN / non-finite codes
    sums.assign(cats.size() + 1, 0.0);
    counts.assign(cats.size() + 1, 0.0);
    auto slot = [&](double code) {
        const int64_t c = category_of(cats, code);
        return c < 0 ? missing : c;
    };
    for (int64_t i = 0; i < t; i++) {
        if (!std::isfinite(tg[i])) continue;
        const int64_t c = slot(row[i]);
        sums[c] += tg[i];
        counts[c] += 1.0;
    }
    auto value = [&](int64_t c) { return (float)((1.0 * mean + sums[c]) / (1.0 + counts[c])); };
    for (int64_t i = 0; i < t; i++) {
        // A missing code before the target starts (or outside its window) is padding.
        dst[i] = std::isnan(tg[i]) && std::isnan(row[i]) ? std::numeric_limits<float>::quiet_NaN() : value(slot(row[i]));
    }
    for (int64_t i = t; i < len; i++) {
        const double code = row[i];
        if (std::isnan(code)) {
            dst[i] = value(missing);
        } else {
            const int64_t c = category_of(cats, code);
            dst[i] = c < 0 ? (float)mean : value(c);
        }
    }
}

}  // namespace

extern "C" int tsfm_timestral_encode_categorical(const tsfm_categorical_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (a->batch < 0 || a->n_cat < 0 || a->t < 1 || a->len < a->t || a->variates < 1)
        return fail(TSFM_E_INVALID, "sizes: batch %d, n_cat %d, t %lld, len %lld, variates %d", a->batch, a->n_cat,
                    (long long)a->t, (long long)a->len, a->variates);
    if (a->row0 < 0 || a->out_rows < 0 || (int64_t)a->row0 + a->n_cat > a->out_rows)
        return fail(TSFM_E_INVALID, "rows %d .. %d outside the %d rows of out", a->row0, a->row0 + a->n_cat, a->out_rows);
    if (a->max_context <= 0) return fail(TSFM_E_INVALID, "max_context %lld", (long long)a->max_context);
    if (a->batch == 0 || a->n_cat == 0) return TSFM_OK;
    if (a->out == nullptr || a->codes == nullptr) return fail(TSFM_E_INVALID, "out and codes are required");
    const bool encode = a->variates == 1;
    if (encode && (a->inputs == nullptr || a->observed == nullptr))
        return fail(TSFM_E_INVALID, "inputs and observed are required with one target variate");

    const int64_t t = a->t, len = a->len;
    std::vector<double> tg((size_t)t), cats, sums, counts;
    for (int64_t s = 0; s < a->batch; s++) {
        if (encode) {  // encodingTarget
            bool started = false;
            float last = 0.f;
            for (int64_t i = 0; i < t; i++) {
                if (a->observed[s * t + i]) {
                    started = true;
                    last = a->inputs[s * t + i];
                }
                const bool in_window = t <= a->max_context || i >= t - a->max_context;
                tg[(size_t)i] = started && in_window ? (double)last : std::numeric_limits<double>::quiet_NaN();
            }
        }
        for (int64_t j = 0; j < a->n_cat; j++) {
            const double* row = a->codes + (s * a->n_cat + j) * len;
            float* dst = a->out + (s * a->out_rows + a->row0 + j) * len;
            if (!encode) {
                for (int64_t i = 0; i < len; i++) dst[i] = (float)row[i];
                continue;
            }
            encode_row(row, tg.data(), t, len, dst, cats, sums, counts);
        }
    }
    return TSFM_OK;
}

// Pointer head (src/head.rs), CPU f64.
#pragma once

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "common.h"

namespace sd {

struct Head {
    std::map<std::string, std::vector<float>> t;
    size_t dim = 0;
    uint64_t id = 0;  // distinct per load (the engine keeps device copies keyed by it)
    void load(const uint8_t* bytes, size_t len);
    std::vector<double> normalize(const float* x, size_t d) const;  // LayerNorm, eps 1e-5
    std::vector<std::vector<double>> project(const char* which, const std::vector<std::vector<double>>& xs,
                                             size_t d) const;
    // Option probabilities from rows [option 0 .. option n-2, answer], each d wide.
    std::vector<double> probs(const float* hidden, size_t n_rows, size_t d, double temperature) const;
};

}  // namespace sd

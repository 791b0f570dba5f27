// RandomPicker.h -- the reference's standalone picker classes
// (src/proxies/RandomPicker.cuh) over the engine's C ABI: same class names,
// constructors and methods.  `use_gpu` is kept for the interface; every pick
// runs on the GPU (trw_pick_index / trw_pick_weights).  The *_batch methods
// go beyond the reference: many picks in one launch.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

class ExponentialIndexRandomPicker {
    bool use_gpu;

public:
    explicit ExponentialIndexRandomPicker(bool use_gpu);
    int pick_random(int start, int end, bool prioritize_end) const;
    int pick_random_with_provided_number(int start, int end, bool prioritize_end,
                                         const double* rand_nums) const;
    std::vector<int32_t> pick_random_batch(const std::vector<int32_t>& starts,
                                           const std::vector<int32_t>& ends, bool prioritize_end,
                                           const double* rand_nums = nullptr) const;
};

class LinearRandomPicker {
    bool use_gpu;

public:
    explicit LinearRandomPicker(bool use_gpu);
    int pick_random(int start, int end, bool prioritize_end) const;
    int pick_random_with_provided_number(int start, int end, bool prioritize_end,
                                         const double* rand_nums) const;
    std::vector<int32_t> pick_random_batch(const std::vector<int32_t>& starts,
                                           const std::vector<int32_t>& ends, bool prioritize_end,
                                           const double* rand_nums = nullptr) const;
};

class UniformRandomPicker {
    bool use_gpu;

public:
    explicit UniformRandomPicker(bool use_gpu);
    int pick_random(int start, int end, bool prioritize_end) const;
    int pick_random_with_provided_number(int start, int end, bool prioritize_end,
                                         const double* rand_nums) const;
    std::vector<int32_t> pick_random_batch(const std::vector<int32_t>& starts,
                                           const std::vector<int32_t>& ends, bool prioritize_end,
                                           const double* rand_nums = nullptr) const;
};

class WeightBasedRandomPicker {
    bool use_gpu;

public:
    explicit WeightBasedRandomPicker(bool use_gpu);
    int pick_random(const double* weights, size_t weights_size, size_t group_start,
                    size_t group_end) const;
    int pick_random_with_provided_number(const double* weights, size_t weights_size,
                                         size_t group_start, size_t group_end,
                                         const double* rand_nums) const;
    int pick_random(const std::vector<double>& cumulative_weights, int group_start,
                    int group_end) const;
    int pick_random_with_provided_number(const std::vector<double>& cumulative_weights,
                                         int group_start, int group_end,
                                         const double* rand_nums) const;
    std::vector<int32_t> pick_random_batch(const std::vector<double>& cumulative_weights,
                                           const std::vector<uint64_t>& group_starts,
                                           const std::vector<uint64_t>& group_ends,
                                           const double* rand_nums = nullptr) const;
};

// RandomPicker.cpp -- standalone pickers over trw_pick_index / trw_pick_weights.
#include "RandomPicker.h"

#include <new>
#include <random>
#include <stdexcept>
#include <string>

#include "trw_engine.h"

namespace {

void check(trw_status st) {
    if (st == TRW_OK) return;
    const std::string msg = trw_last_error();
    switch (st) {
        case TRW_ERR_INVALID_ARGUMENT: throw std::invalid_argument(msg);
        case TRW_ERR_OUT_OF_MEMORY: throw std::bad_alloc();
        default: throw std::runtime_error(msg);
    }
}

// pick_random draws from a fresh generator on every call
// (common/random_gen.cuh:27-45 of the reference): a fresh Philox key here.
uint64_t fresh_seed() {
    std::random_device rd;
    return (static_cast<uint64_t>(rd()) << 32) | rd();
}

int pick_one(int picker, int start, int end, bool prioritize_end, const double* r) {
    int32_t out = -1;
    check(trw_pick_index(-1, picker, &start, &end, 1, prioritize_end ? 1 : 0, r,
                         r ? 0 : fresh_seed(), &out));
    return out;
}

std::vector<int32_t> pick_many(int picker, const std::vector<int32_t>& starts,
                               const std::vector<int32_t>& ends, bool prioritize_end,
                               const double* r) {
    if (starts.size() != ends.size())
        throw std::invalid_argument("starts and ends must have the same length");
    std::vector<int32_t> out(starts.size());
    check(trw_pick_index(-1, picker, starts.data(), ends.data(), starts.size(),
                         prioritize_end ? 1 : 0, r, r ? 0 : fresh_seed(), out.data()));
    return out;
}

}  // namespace

ExponentialIndexRandomPicker::ExponentialIndexRandomPicker(bool g) : use_gpu(g) {}
int ExponentialIndexRandomPicker::pick_random(int start, int end, bool prioritize_end) const {
    return pick_one(TRW_PICKER_EXPONENTIAL_INDEX, start, end, prioritize_end, nullptr);
}
int ExponentialIndexRandomPicker::pick_random_with_provided_number(int start, int end,
                                                                   bool prioritize_end,
                                                                   const double* r) const {
    return pick_one(TRW_PICKER_EXPONENTIAL_INDEX, start, end, prioritize_end, r);
}
std::vector<int32_t> ExponentialIndexRandomPicker::pick_random_batch(
    const std::vector<int32_t>& starts, const std::vector<int32_t>& ends, bool prioritize_end,
    const double* r) const {
    return pick_many(TRW_PICKER_EXPONENTIAL_INDEX, starts, ends, prioritize_end, r);
}

LinearRandomPicker::LinearRandomPicker(bool g) : use_gpu(g) {}
int LinearRandomPicker::pick_random(int start, int end, bool prioritize_end) const {
    return pick_one(TRW_PICKER_LINEAR, start, end, prioritize_end, nullptr);
}
int LinearRandomPicker::pick_random_with_provided_number(int start, int end, bool prioritize_end,
                                                         const double* r) const {
    return pick_one(TRW_PICKER_LINEAR, start, end, prioritize_end, r);
}
std::vector<int32_t> LinearRandomPicker::pick_random_batch(const std::vector<int32_t>& starts,
                                                           const std::vector<int32_t>& ends,
                                                           bool prioritize_end,
                                                           const double* r) const {
    return pick_many(TRW_PICKER_LINEAR, starts, ends, prioritize_end, r);
}

UniformRandomPicker::UniformRandomPicker(bool g) : use_gpu(g) {}
int UniformRandomPicker::pick_random(int start, int end, bool prioritize_end) const {
    return pick_one(TRW_PICKER_UNIFORM, start, end, prioritize_end, nullptr);
}
int UniformRandomPicker::pick_random_with_provided_number(int start, int end, bool prioritize_end,
                                                          const double* r) const {
    return pick_one(TRW_PICKER_UNIFORM, start, end, prioritize_end, r);
}
std::vector<int32_t> UniformRandomPicker::pick_random_batch(const std::vector<int32_t>& starts,
                                                            const std::vector<int32_t>& ends,
                                                            bool prioritize_end,
                                                            const double* r) const {
    return pick_many(TRW_PICKER_UNIFORM, starts, ends, prioritize_end, r);
}

WeightBasedRandomPicker::WeightBasedRandomPicker(bool g) : use_gpu(g) {}
int WeightBasedRandomPicker::pick_random(const double* weights, size_t weights_size,
                                         size_t group_start, size_t group_end) const {
    return pick_random_with_provided_number(weights, weights_size, group_start, group_end,
                                            nullptr);
}
int WeightBasedRandomPicker::pick_random_with_provided_number(const double* weights,
                                                              size_t weights_size,
                                                              size_t group_start,
                                                              size_t group_end,
                                                              const double* r) const {
    int32_t out = -1;
    const uint64_t gs = group_start, ge = group_end;
    check(trw_pick_weights(-1, weights, weights_size, &gs, &ge, 1, r, r ? 0 : fresh_seed(), &out));
    return out;
}
int WeightBasedRandomPicker::pick_random(const std::vector<double>& w, int group_start,
                                         int group_end) const {
    // int -> size_t as in the reference (a negative start wraps and is rejected)
    return pick_random(w.data(), w.size(), static_cast<size_t>(group_start),
                       static_cast<size_t>(group_end));
}
int WeightBasedRandomPicker::pick_random_with_provided_number(const std::vector<double>& w,
                                                              int group_start, int group_end,
                                                              const double* r) const {
    return pick_random_with_provided_number(w.data(), w.size(), static_cast<size_t>(group_start),
                                            static_cast<size_t>(group_end), r);
}
std::vector<int32_t> WeightBasedRandomPicker::pick_random_batch(
    const std::vector<double>& w, const std::vector<uint64_t>& starts,
    const std::vector<uint64_t>& ends, const double* r) const {
    if (starts.size() != ends.size())
        throw std::invalid_argument("group_starts and group_ends must have the same length");
    std::vector<int32_t> out(starts.size());
    check(trw_pick_weights(-1, w.data(), w.size(), starts.data(), ends.data(), starts.size(), r,
                           r ? 0 : fresh_seed(), out.data()));
    return out;
}

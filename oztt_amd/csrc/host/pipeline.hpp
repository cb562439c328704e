// Running a backend's recorded device steps, with the evaluation hooks when they are active
// (reference evaluation_hooks.hpp:56-219): the steps are stream-ordered launches on the library's
// stream with no host synchronization between them, so the same list is issued once for the call
// and replayed for the whole-pass timing.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

#include "evaluation.hpp"
#include "oz_hip.h"

namespace ozTTgemm::detail {

struct Step {
    evaluation::Phase phase;
    std::function<void()> issue;
};

// Issues `steps` (timing each phase, then replaying the whole pass and the product steps, those of
// phase Gemm, under an active evaluation Scope), reads back the `count` result values of `out` into
// `host` (none for a result that stays on the device) and the two range flags, and throws
// std::runtime_error for a set flag (scale.hpp:187-208).
// product_ops / partial_products describe the product phase for the evaluation record.
void run_pipeline(oz_dev* dev, const std::vector<Step>& steps, const double* out, double* host, std::size_t count,
                  const std::uint32_t* flags, double product_ops, unsigned partial_products);

}  // namespace ozTTgemm::detail

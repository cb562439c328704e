// Running a backend's recorded device steps, with the evaluation hooks when they are active
// (reference evaluation_hooks.hpp:56-219): the steps are stream-ordered launches on the library's
// stream with no host synchronization between them, so the same list is issued once for the call
// and replayed for the whole-pass timing.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

#include "backend.hpp"
#include "evaluation.hpp"
#include "oz_hip.h"

namespace ozTTgemm::detail {

struct Step {
    evaluation::Phase phase;
    std::function<void()> issue;
};

// A device region that one pass writes (every intermediate and the output, never an input).
// Sizes are whole 32-bit words.
struct Written {
    void* p;
    std::size_t bytes;
};

// What one call's pass consists of, stated by the backend from its configuration (not from the
// step list): the device steps it issues per phase, and the regions they write.
struct PassShape {
    unsigned steps[evaluation::PhaseCount] = {};
    std::vector<Written> written;
};

// Issues `steps` (timing each phase, then checking and replaying the whole pass under an active
// evaluation Scope with repeats), reads back the `count` result values of `out` into `host` (none
// when host is null: the result stays on the device) and the two range flags of the first pass (the
// slot of `ws` its scale step used), and throws std::runtime_error for a set flag
// (scale.hpp:187-208). `out` holds `count` values in any case.
//
// The whole-pass check (evaluation_hooks.hpp:175-211): every region of `shape.written` (every
// intermediate and the output; the range flags are ORed into, not written, and have their own slots)
// is filled with a sentinel, which must then be read back from the output; one checking replay issues the
// steps, counted per phase against shape.steps; its output and the output after the timed replays
// must both be bit-identical to the first pass. Only then is whole_checked set.
// product_ops / partial_products describe the product phase for the evaluation record.
void run_pipeline(oz_dev* dev, const std::vector<Step>& steps, const PassShape& shape, const double* out,
                  double* host, std::size_t count, const Workspace& ws, double product_ops,
                  unsigned partial_products);

}  // namespace ozTTgemm::detail

// See pipeline.hpp.
#include "pipeline.hpp"

#include <cstring>
#include <stdexcept>
#include <string>

#include "backend.hpp"

namespace ozTTgemm::detail {

namespace ev = ::ozTTgemm::evaluation;

void run_pipeline(oz_dev* dev, const std::vector<Step>& steps, const double* out, double* host, std::size_t count,
                  const std::uint32_t* flags, double product_ops, unsigned partial_products) {
    ev::Settings* es = ev::active();
    // Per-phase device times: events around every step (slots 24 + 2i, 25 + 2i), summed by phase.
    // The events are read after the pass, so each step needs its own pair.
    constexpr int kFirstSlot = 24, kSlots = 64;
    const bool step_events = es && kFirstSlot + 2 * steps.size() <= kSlots;
    auto timed_pass = [&](double* phase_ms) {
        for (std::size_t i = 0; i < steps.size(); i++) {
            device_check(dev, oz_event_record(dev, kFirstSlot + 2 * (int)i), "event");
            steps[i].issue();
            device_check(dev, oz_event_record(dev, kFirstSlot + 2 * (int)i + 1), "event");
        }
        for (std::size_t i = 0; i < steps.size(); i++) {
            float ms = 0;
            device_check(dev, oz_event_elapsed_ms(dev, kFirstSlot + 2 * (int)i, kFirstSlot + 2 * (int)i + 1, &ms),
                         "event time");
            phase_ms[steps[i].phase] += ms;
        }
    };
    if (!es) {
        for (auto& s : steps) s.issue();
    } else {
        // first pass; its phase times stand unless replays follow (then the warm replays replace them)
        for (int ph = 0; ph < ev::PhaseCount; ph++) es->phase_ms[ph] = 0;
        if (step_events)
            timed_pass(es->phase_ms);
        else
            for (auto& s : steps) s.issue();
        es->partial_products = partial_products;
        es->product_ops = product_ops;
        es->gemm_launches = 0;
        for (auto& s : steps) es->gemm_launches += s.phase == ev::Gemm;
    }
    if (count) device_check(dev, oz_memcpy_d2h(dev, host, out, sizeof(double) * count), "read C");
    std::uint32_t fl[2];
    device_check(dev, oz_memcpy_d2h(dev, fl, flags, sizeof fl), "read flags");

    if (es && es->repeats > 0) {
        // whole pass: warm up, then `repeats` replays between two events; then the product step
        // alone, for its average launch time
        for (int w = 0; w < es->warmup; w++)
            for (auto& s : steps) s.issue();
        device_check(dev, oz_event_record(dev, 20), "event");
        for (int r = 0; r < es->repeats; r++)
            for (auto& s : steps) s.issue();
        device_check(dev, oz_event_record(dev, 21), "event");
        float ms = 0;
        device_check(dev, oz_event_elapsed_ms(dev, 20, 21, &ms), "event time");
        es->whole_ms = ms / es->repeats;
        std::vector<double> again(count);
        if (count) device_check(dev, oz_memcpy_d2h(dev, again.data(), out, sizeof(double) * count), "read C");
        es->whole_checked = count && std::memcmp(again.data(), host, sizeof(double) * count) == 0;
        device_check(dev, oz_event_record(dev, 22), "event");
        for (int r = 0; r < es->repeats; r++)
            for (auto& s : steps)
                if (s.phase == ev::Gemm) s.issue();
        device_check(dev, oz_event_record(dev, 23), "event");
        device_check(dev, oz_event_elapsed_ms(dev, 22, 23, &ms), "event time");
        es->gemm_launch_ms = ms / es->repeats;
        // warm phase times: the average of up to 5 more passes with events between the steps
        if (step_events) {
            const int passes = es->repeats < 5 ? es->repeats : 5;
            double acc[ev::PhaseCount] = {};
            for (int r = 0; r < passes; r++) timed_pass(acc);
            for (int ph = 0; ph < ev::PhaseCount; ph++) es->phase_ms[ph] = acc[ph] / passes;
        }
    }
    // range flags of the scaling stage; the host validation rejects these inputs first, so they only
    // fire if the device disagrees with it
    for (int t = 0; t < 2; t++)
        if (fl[t]) {
            const char* what = t == 0 ? "rows of A" : "columns of B";
            if (fl[t] & 4u) throw std::runtime_error(std::string("the ") + what + " contain Inf or NaN");
            if (fl[t] & 2u) throw std::runtime_error(std::string("a maximum of the ") + what + " is below 2^-126");
            throw std::runtime_error(std::string("a maximum of the ") + what + " exceeds the BF16 range");
        }
}

}  // namespace ozTTgemm::detail

// See pipeline.hpp.
#include "pipeline.hpp"

#include <cstring>
#include <stdexcept>
#include <string>

#include "backend.hpp"

namespace ozTTgemm::detail {

namespace ev = ::ozTTgemm::evaluation;

std::vector<double> run_pipeline(oz_dev* dev, const std::vector<Step>& steps, std::size_t gemm_step,
                                 const double* out, std::size_t count, const std::uint32_t* flags,
                                 double product_ops, unsigned partial_products) {
    ev::Settings* es = ev::active();
    if (!es) {
        for (auto& s : steps) s.issue();
    } else {
        // first pass: phase times with events on the stream (slots 2*phase, 2*phase+1)
        for (auto& s : steps) {
            device_check(dev, oz_event_record(dev, 2 * s.phase), "event");
            s.issue();
            device_check(dev, oz_event_record(dev, 2 * s.phase + 1), "event");
        }
        for (int ph = 0; ph < ev::PhaseCount; ph++) es->phase_ms[ph] = 0;
        for (auto& s : steps) {
            float ms = 0;
            device_check(dev, oz_event_elapsed_ms(dev, 2 * s.phase, 2 * s.phase + 1, &ms), "event time");
            es->phase_ms[s.phase] += ms;
        }
        es->partial_products = partial_products;
        es->product_ops = product_ops;
        es->gemm_launches = 1;
    }
    std::vector<double> values(count);
    device_check(dev, oz_memcpy_d2h(dev, values.data(), out, sizeof(double) * count), "read C");
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
        device_check(dev, oz_memcpy_d2h(dev, again.data(), out, sizeof(double) * count), "read C");
        es->whole_checked = std::memcmp(again.data(), values.data(), sizeof(double) * count) == 0;
        device_check(dev, oz_event_record(dev, 22), "event");
        for (int r = 0; r < es->repeats; r++) steps[gemm_step].issue();
        device_check(dev, oz_event_record(dev, 23), "event");
        device_check(dev, oz_event_elapsed_ms(dev, 22, 23, &ms), "event time");
        es->gemm_launch_ms = ms / es->repeats;
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
    return values;
}

}  // namespace ozTTgemm::detail

// See pipeline.hpp.
#include "pipeline.hpp"

#include <cstring>
#include <stdexcept>
#include <string>

#include "backend.hpp"

namespace ozTTgemm::detail {

namespace ev = ::ozTTgemm::evaluation;

namespace {

// Written into every region a pass writes before the checking replay. As a double, the doubled
// word is a NaN, which no reconstruction produces, so a value that survives is never mistaken for
// a result.
constexpr std::uint32_t kSentinel = 0x7FF4DEADu;

std::vector<double> read_back(oz_dev* dev, const double* out, std::size_t count) {
    std::vector<double> v(count);
    if (count) device_check(dev, oz_memcpy_d2h(dev, v.data(), out, sizeof(double) * count), "read C");
    return v;
}

bool same_bits(const std::vector<double>& x, const double* y, std::size_t count) {
    return x.size() == count && (count == 0 || std::memcmp(x.data(), y, sizeof(double) * count) == 0);
}

bool whole_counts_match(const ev::Settings& s) {
    for (int ph = 0; ph < ev::PhaseCount; ph++)
        if (s.whole_steps[ph] != s.expected_steps[ph]) return false;
    return true;
}

}  // namespace

void run_pipeline(oz_dev* dev, const std::vector<Step>& steps, const PassShape& shape, const double* out,
                  double* host, std::size_t count, const Workspace& ws, double product_ops,
                  unsigned partial_products) {
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
        es->whole_checked = false;
        es->whole_sentinel = false;
        for (int ph = 0; ph < ev::PhaseCount; ph++) {
            es->whole_steps[ph] = 0;
            es->expected_steps[ph] = shape.steps[ph];
        }
    }
    if (host && count) device_check(dev, oz_memcpy_d2h(dev, host, out, sizeof(double) * count), "read C");
    std::uint32_t fl[2];
    device_check(dev, oz_memcpy_d2h(dev, fl, ws.last_flags(), sizeof fl), "read flags");

    // the first pass's result (when it is not in `host`), the reference of every replay
    std::vector<double> whole_ref;
    if (es && es->repeats > 0) {
        std::vector<double> first;
        const double* ref = host;
        if (!host) {
            first = read_back(dev, out, count);
            ref = first.data();
        }
        // 1. sentinel in every region the pass writes; the output must read back as sentinel
        for (const Written& w : shape.written)
            device_check(dev, oz_fill_u32(dev, w.p, kSentinel, w.bytes / 4), "sentinel fill");
        std::vector<double> got = read_back(dev, out, count);
        bool filled = count > 0;
        for (std::size_t i = 0; filled && i < count; i++) {
            std::uint64_t u;
            std::memcpy(&u, &got[i], 8);
            filled = u == ((std::uint64_t)kSentinel << 32 | kSentinel);
        }
        // 2. one checking replay, its steps counted per phase (the checker's self-test can leave out
        //    one phase; that run then stops after the check and times nothing)
        for (auto& s : steps) {
            if ((int)s.phase == es->replay_drop_phase) continue;
            s.issue();
            es->whole_steps[s.phase]++;
        }
        got = read_back(dev, out, count);
        es->whole_sentinel = filled && same_bits(got, ref, count);
        if (!host) whole_ref = std::move(first);
        es->whole_ms = 0;
        es->gemm_launch_ms = 0;
        // after the self-test's incomplete replay, one whole pass restores the result on the device
        if (es->replay_drop_phase >= 0)
            for (auto& s : steps) s.issue();
    }
    if (es && es->repeats > 0 && es->replay_drop_phase < 0) {
        // 3. whole pass: warm up, then `repeats` replays between two events; the output must still
        //    be the first pass's
        //    The product steps of the timed passes are bracketed by events too (slots 24.. while they
        //    last: every pass whose product steps fit), which gives the products' time per pass as
        //    they run inside the whole pass (an event marker costs no measurable time).
        for (int w = 0; w < es->warmup; w++)
            for (auto& s : steps) s.issue();
        int slot = kFirstSlot, timed_passes = 0;
        std::size_t gemm_steps = 0;
        for (auto& s : steps) gemm_steps += s.phase == ev::Gemm;
        device_check(dev, oz_event_record(dev, 20), "event");
        for (int r = 0; r < es->repeats; r++) {
            const bool mark = slot + 2 * gemm_steps <= (std::size_t)kSlots;
            for (auto& s : steps) {
                if (mark && s.phase == ev::Gemm) device_check(dev, oz_event_record(dev, slot++), "event");
                s.issue();
                if (mark && s.phase == ev::Gemm) device_check(dev, oz_event_record(dev, slot++), "event");
            }
            timed_passes += mark;
        }
        device_check(dev, oz_event_record(dev, 21), "event");
        float ms = 0;
        device_check(dev, oz_event_elapsed_ms(dev, 20, 21, &ms), "event time");
        es->whole_ms = ms / es->repeats;
        double gemm_ms = 0;
        for (int e = kFirstSlot; e < slot; e += 2) {
            device_check(dev, oz_event_elapsed_ms(dev, e, e + 1, &ms), "event time");
            gemm_ms += ms;
        }
        es->gemm_launch_ms = timed_passes ? gemm_ms / timed_passes : 0.0;
        const std::vector<double> last = read_back(dev, out, count);
        es->whole_checked = es->whole_sentinel && whole_counts_match(*es) &&
                            same_bits(last, host ? host : whole_ref.data(), count);
        // 4. warm phase times: the average of up to 5 more passes with events between the steps
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

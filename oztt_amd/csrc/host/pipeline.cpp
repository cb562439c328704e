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
    // Event slots: 20 and 21 bracket the timed replays; from 24 on, a pair of slots around each step
    // that is timed on its own. Events are read only after every pass is issued, so no host wait
    // leaves the device idle (and its clock falling) between the passes.
    constexpr int kFirstSlot = 24, kSlots = OZ_EVENT_SLOTS;
    struct Marked {
        int phase, slot;
    };
    // one pass; each step that `mark` selects between its own pair of events (slots from `slot` on)
    auto marked_pass = [&](auto&& mark, int& slot, std::vector<Marked>& marked) {
        for (auto& s : steps) {
            const bool m = mark(s);
            if (m) {
                device_check(dev, oz_event_record(dev, slot), "event");
                marked.push_back({(int)s.phase, slot});
            }
            s.issue();
            if (m) {
                device_check(dev, oz_event_record(dev, slot + 1), "event");
                slot += 2;
            }
        }
    };
    auto elapsed = [&](int a, int b) {
        float ms = 0;
        device_check(dev, oz_event_elapsed_ms(dev, a, b, &ms), "event time");
        return (double)ms;
    };
    auto every = [](const Step&) { return true; };
    const bool step_events = es && kFirstSlot + 2 * steps.size() <= (std::size_t)kSlots;
    if (!es) {
        for (auto& s : steps) s.issue();
    } else {
        // first pass; its phase times stand unless replays follow (then the warm replays replace them)
        for (int ph = 0; ph < ev::PhaseCount; ph++) es->phase_ms[ph] = 0;
        if (step_events) {
            int slot = kFirstSlot;
            std::vector<Marked> marked;
            marked_pass(every, slot, marked);
            for (const Marked& m : marked) es->phase_ms[m.phase] += elapsed(m.slot, m.slot + 1);
        } else {
            for (auto& s : steps) s.issue();
        }
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
        for (int w = 0; w < es->warmup; w++)
            for (auto& s : steps) s.issue();
        device_check(dev, oz_event_record(dev, 20), "event");
        for (int r = 0; r < es->repeats; r++)
            for (auto& s : steps) s.issue();
        device_check(dev, oz_event_record(dev, 21), "event");
        // 4. right after them, with no wait: up to `repeats` passes whose product launches are timed
        //    (the products' time per pass as they run inside whole passes; kept out of the timed
        //    region all the same), then up to 5 passes with events around every step (the warm phase
        //    times). Slots [24, 140) take the products, [140, 256) the phases.
        constexpr int kPhaseSlot = kFirstSlot + (kSlots - kFirstSlot) / 2;
        std::size_t gemm_steps = 0;
        for (auto& s : steps) gemm_steps += s.phase == ev::Gemm;
        //    A product step is timed by its kernels' own dispatches (oz_time_products_begin), not by
        //    markers around it: those would add the dispatch latency they bracket, a fifth of a
        //    20 µs launch. A step that launched no product kernel counts as zero.
        int slot = kFirstSlot, gemm_passes = 0;
        std::vector<Marked> gm;
        for (int r = 0; r < es->repeats && slot + 2 * gemm_steps <= (std::size_t)kPhaseSlot; r++, gemm_passes++)
            for (auto& s : steps) {
                if (s.phase != ev::Gemm) {
                    s.issue();
                    continue;
                }
                device_check(dev, oz_time_products_begin(dev, slot, slot + 1), "product timing");
                struct EndRequest {  // a step that throws leaves no request behind on the handle
                    oz_dev* d;
                    ~EndRequest() { oz_time_products_end(d, nullptr); }
                } guard{dev};
                s.issue();
                int launched = 0;
                device_check(dev, oz_time_products_end(dev, &launched), "product timing");
                if (launched)
                    gm.push_back({(int)s.phase, slot});
                slot += 2;
            }
        int pslot = kPhaseSlot, phase_passes = 0;
        std::vector<Marked> pm;
        for (int r = 0; r < es->repeats && r < 5 && pslot + 2 * steps.size() <= (std::size_t)kSlots;
             r++, phase_passes++)
            marked_pass(every, pslot, pm);
        es->whole_ms = elapsed(20, 21) / es->repeats;
        double gemm_ms = 0;
        for (const Marked& m : gm) gemm_ms += elapsed(m.slot, m.slot + 1);
        es->gemm_launch_ms = gemm_passes ? gemm_ms / gemm_passes : 0.0;
        if (phase_passes) {
            double acc[ev::PhaseCount] = {};
            for (const Marked& m : pm) acc[m.phase] += elapsed(m.slot, m.slot + 1);
            for (int ph = 0; ph < ev::PhaseCount; ph++) es->phase_ms[ph] = acc[ph] / phase_passes;
        }
        const std::vector<double> last = read_back(dev, out, count);
        es->whole_checked = es->whole_sentinel && whole_counts_match(*es) &&
                            same_bits(last, host ? host : whole_ref.data(), count);
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

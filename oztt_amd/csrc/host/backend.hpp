// Interface between the public Context (context.cpp) and the backends (one per scheme and format),
// and the device handle shared by them. Mirrors the reference's backend_interface.hpp:14-35: a
// backend receives the validated, zero-padded problem and returns the padded result.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include <ozTTgemm/ozTTgemm.hpp>

#include "oz_hip.h"

namespace ozTTgemm::detail {

// Throws std::runtime_error with the device layer's message when a C-ABI call fails.
void device_check(oz_dev* dev, int status, const char* what);

// Device allocations of one GPU kept by the Context between calls, grown on demand (the reference
// rebuilds its buffers per call, README.md:81-85; reusing them avoids hipMalloc in repeated calls),
// and page-locked host staging buffers for the operands and the result, kept the same way.
class Workspace {
public:
    explicit Workspace(oz_dev* dev) : dev_(dev) {}
    ~Workspace();
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    // Device buffer of at least `bytes` for role `slot` (contents undefined).
    void* get(int slot, std::size_t bytes);
    // Page-locked host buffer of at least `bytes` for role `slot` (contents undefined); ordinary
    // memory if page-locked memory is refused.
    void* host(int slot, std::size_t bytes);
    // Device bytes held by the slots, and the release of one slot's device buffer.
    std::size_t held() const;
    void release(int slot);
    void release_all();

    // The range flags of the scaling stage (two device words per pass), kept in two slots so that
    // no launch has to clear them: a pass ORs its flags into one slot while its scale launch zeroes
    // the other, which the next pass then uses. flag_slots() gives this pass's slot (`use`) and the
    // one to zero (`clear`); flags_issued() moves on once that scale launch has been issued (a pass
    // whose scale launch failed uses the same slots again); last_flags() is the slot of the scale
    // launch issued last. Both slots start at zero.
    struct FlagSlots {
        std::uint32_t* use;
        std::uint32_t* clear;
    };
    FlagSlots flag_slots();
    void flags_issued() { parity_ ^= 1u; }
    const std::uint32_t* last_flags() const { return flags_ + 2 * (parity_ ^ 1u); }

private:
    struct Buf {
        void* p = nullptr;
        std::size_t size = 0;
        bool pinned = false;
    };
    void free_host(Buf& b);
    oz_dev* dev_;
    std::vector<Buf> bufs_, host_;
    std::uint32_t* flags_ = nullptr;  // 2 slots x 2 words
    unsigned parity_ = 0;
};

// Host staging slots.
enum HostSlot { kHostA = 0, kHostB, kHostC };


// The opened GPU (the reference's Device, backend_interface.hpp:14).
struct Device {
    oz_dev* dev = nullptr;
    std::unique_ptr<Workspace> ws;
};

// Row bands (the reference's row bands when device memory runs short, ozaki2/plan.hpp:386-444):
// the rows of A and C per band, either all M, or the largest multiple of 256 for which
// `fixed` bytes plus `per_row` bytes per padded row fit in the device memory left beside the other
// slots of the workspace (the slots listed in `band_slots` are released to make room). An active
// evaluation Scope may cap the band (Settings::max_band_rows). std::runtime_error when not even
// 256 rows fit.
std::uint32_t band_rows(Device& D, std::uint32_t M, std::size_t fixed, std::size_t per_row,
                        std::initializer_list<int> band_slots);

// One GEMM after validation and zero padding: A is m x k and B is k x n, row-major, with m and n
// multiples of 64 and k a multiple of 32 (backend_interface.hpp:21-26). The operands are in the
// workspace's page-locked staging buffers (a, b: what the planner reads).
// Resident operands (Context::Matrix) add device copies in the same padded layout (a_dev, b_dev:
// the backend then uploads nothing) and may bring the plan made for them earlier (plan: the
// planner is skipped, and a and b may be null); c_dev receives the padded m x n result on the
// device instead of the host staging.
struct Problem {
    std::uint32_t m, n, k;
    const double* a;
    const double* b;
    const Options& options;
    const double* a_dev = nullptr;
    const double* b_dev = nullptr;
    double* c_dev = nullptr;
    std::shared_ptr<const void> plan;  // a Plan1 (scheme I) or Plan2 (scheme II) of this backend
};

struct Output {
    const double* values;  // padded m x n, row-major, in the workspace's host staging (kHostC); null with c_dev
    Info info;
    std::shared_ptr<const void> plan;  // the plan the call ran (for the Context's cache)
};

using Backend = Output (*)(Device&, const Problem&);

// Throws std::invalid_argument for a (format, scheme) pair that this build does not implement.
Backend backend_for(Format format, Scheme scheme);
bool scheme_available(Format format, Scheme scheme) noexcept;

// Backends.
Output ozaki2_run(Device& dev, const Problem& p);
Output ozaki1_run(Device& dev, const Problem& p);

}  // namespace ozTTgemm::detail

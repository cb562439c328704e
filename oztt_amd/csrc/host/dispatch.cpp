// (format, scheme) -> backend, format names, availability; the device workspace. Semantics of the
// reference's dispatch.cpp:18-51: formats that are not built report is_available() == false.
#include <new>
#include <stdexcept>

#include "backend.hpp"
#include "evaluation.hpp"

#include <algorithm>

namespace ozTTgemm::detail {

void device_check(oz_dev* dev, int status, const char* what) {
    if (status == OZ_OK) return;
    throw std::runtime_error(std::string(what) + ": " + oz_last_error(dev));
}

Workspace::~Workspace() {
    release_all();
    if (flags_) (void)oz_dev_free(dev_, flags_);
}

Workspace::FlagSlots Workspace::flag_slots() {
    if (!flags_) {
        void* p = nullptr;
        device_check(dev_, oz_dev_malloc(dev_, 4 * sizeof(std::uint32_t), &p), "device allocation");
        flags_ = static_cast<std::uint32_t*>(p);
        parity_ = 0;
        device_check(dev_, oz_fill_u32(dev_, flags_, 0u, 4), "flags");  // stream-ordered before any use
    }
    return {flags_ + 2 * parity_, flags_ + 2 * (parity_ ^ 1u)};
}

void* Workspace::get(int slot, std::size_t bytes) {
    if (slot < 0) throw std::logic_error("workspace slot");
    if ((std::size_t)slot >= bufs_.size()) bufs_.resize(slot + 1);
    Buf& b = bufs_[slot];
    bytes = (bytes + 255) & ~std::size_t(255);
    if (b.size < bytes) {
        if (b.p) device_check(dev_, oz_dev_free(dev_, b.p), "hipFree");
        b.p = nullptr;
        b.size = 0;
        void* p = nullptr;
        device_check(dev_, oz_dev_malloc(dev_, bytes, &p), "device allocation");
        b.p = p;
        b.size = bytes;
    }
    return bufs_[slot].p;
}

void* Workspace::host(int slot, std::size_t bytes) {
    if (slot < 0) throw std::logic_error("host staging slot");
    if ((std::size_t)slot >= host_.size()) host_.resize(slot + 1);
    Buf& b = host_[slot];
    bytes = (bytes + 4095) & ~std::size_t(4095);
    if (b.size < bytes) {
        free_host(b);
        void* p = nullptr;
        if (oz_host_malloc(dev_, bytes, &p) == OZ_OK) {
            b.pinned = true;
        } else {
            // page-locked memory refused (limits or exhaustion): ordinary memory works the same,
            // only the copies are slower; std::bad_alloc when even that runs out
            p = ::operator new(bytes);
            b.pinned = false;
        }
        b.p = p;
        b.size = bytes;
    }
    return b.p;
}

void Workspace::free_host(Buf& b) {
    if (b.p) {
        if (b.pinned)
            (void)oz_host_free(dev_, b.p);
        else
            ::operator delete(b.p);
    }
    b.p = nullptr;
    b.size = 0;
}

std::size_t Workspace::held() const {
    std::size_t n = 0;
    for (const auto& b : bufs_) n += b.size;
    return n;
}

void Workspace::release(int slot) {
    if (slot < 0 || (std::size_t)slot >= bufs_.size()) return;
    Buf& b = bufs_[slot];
    if (b.p) (void)oz_dev_free(dev_, b.p);
    b.p = nullptr;
    b.size = 0;
}

std::uint32_t band_rows(Device& D, std::uint32_t M, std::size_t fixed, std::size_t per_row,
                        std::initializer_list<int> band_slots) {
    const std::uint32_t Mg = (M + 255) / 256 * 256;
    std::uint32_t rows = M;
    std::size_t free_b = 0, total_b = 0;
    device_check(D.dev, oz_mem_info(D.dev, &free_b, &total_b), "device memory");
    // bytes available: free now plus what the workspace holds (its slots are reallocated as needed),
    // less a margin for the runtime
    const std::size_t margin = std::max<std::size_t>(total_b / 64, std::size_t(1) << 30);
    std::size_t avail = free_b + D.ws->held();
    avail = avail > margin ? avail - margin : 0;
    if (fixed + per_row * (std::size_t)Mg > avail) {
        for (int s : band_slots) D.ws->release(s);
        if (fixed + 256 * per_row > avail)
            throw std::runtime_error("the problem does not fit in device memory, not even in row bands of 256 rows");
        rows = (std::uint32_t)std::min<std::size_t>((avail - fixed) / per_row / 256 * 256, Mg);
    }
    if (const ::ozTTgemm::evaluation::Settings* es = ::ozTTgemm::evaluation::active())
        if (es->max_band_rows > 0) rows = std::min(rows, std::max(256u, es->max_band_rows / 256 * 256));
    return std::min(rows, M);
}

void Workspace::release_all() {
    for (auto& b : bufs_)
        if (b.p) (void)oz_dev_free(dev_, b.p);
    bufs_.clear();
    for (auto& b : host_) free_host(b);
    host_.clear();
}

// Every format runs with both schemes. Scheme I runs every format's digits (int8 values) on the INT8
// matrix cores; Scheme II runs FP8 on the FP8 matrix cores and every other format with INT8 residues
// (the formats without their own MI355X matrix instructions, and BF16/FP16, whose matrix rate is half
// the INT8 rate: see plan_scheme2).
bool scheme_available(Format format, Scheme scheme) noexcept {
    if ((int)format < 0 || (int)format > (int)Format::BFP2) return false;
    return scheme == Scheme::I || scheme == Scheme::II;
}

Backend backend_for(Format format, Scheme scheme) {
    if (scheme == Scheme::I && scheme_available(format, scheme)) return ozaki1_run;
    if (scheme == Scheme::II && scheme_available(format, scheme)) return ozaki2_run;
    throw std::invalid_argument("requested format was not built");
}

}  // namespace ozTTgemm::detail

namespace ozTTgemm {

bool is_available(Format format) noexcept {
    return detail::scheme_available(format, Scheme::I) || detail::scheme_available(format, Scheme::II);
}

const char* format_name(Format format) noexcept {
    switch (format) {
    case Format::BF16: return "BF16";
    case Format::FP16: return "FP16";
    case Format::TF32: return "TF32";
    case Format::BFP8: return "BFP8";
    case Format::FP8: return "FP8";
    case Format::INT8: return "INT8";
    case Format::BFP4: return "BFP4";
    case Format::BFP2: return "BFP2";
    default: return "unknown";
    }
}

}  // namespace ozTTgemm

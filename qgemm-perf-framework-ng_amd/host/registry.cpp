// Kernel catalogue of the standalone runner (pfng_bench). Entries keep their
// registration order, which is the order `--list` prints and `--kernel all`
// runs; an id index makes lookups independent of the catalogue's size.
//
// Registration is fail-closed, as the reference's is (kernel_registry.cpp:18-33):
// a malformed entry is a programming error in an adapter, so the process stops
// at start-up instead of running with a partial catalogue.
#include "registry.h"

#include <cstdio>
#include <cstdlib>
#include <string>
#include <unordered_map>

namespace pfng::bench {

namespace {

struct Catalogue {
    std::vector<KernelRegistration> entries;
    std::unordered_map<std::string, size_t> index_of;  // id -> position in entries
};

Catalogue &catalogue() {
    static Catalogue instance;
    return instance;
}

bool has_every_callback(const KernelCallbacks &cb) {
    return cb.peak_performance && cb.validate && cb.prepare && cb.reset && cb.run && cb.export_output &&
           cb.checksum && cb.destroy;
}

// nullptr when the entry can be added, else what is wrong with it
const char *defect_of(const KernelRegistration &entry) {
    if (entry.id.empty()) return "the kernel id is empty";
    if (entry.name.empty()) return "the display name is empty";
    if (!has_every_callback(entry.callbacks)) return "the callback table has a null entry (all eight are required)";
    if (static_cast<size_t>(entry.quantization) >= static_cast<size_t>(QuantizationType::Count))
        return "the quantization type is out of range";
    if (catalogue().index_of.count(std::string(entry.id))) return "another kernel already uses this id";
    return nullptr;
}

}  // namespace

std::string_view quantization_name(QuantizationType type) {
    static constexpr std::string_view kNames[] = {"WeightQ4_0ActivationQ8_0", "WeightQ4_KActivationQ8_K",
                                                  "WeightIQ2_XXSActivationQ8_K"};
    const size_t i = static_cast<size_t>(type);
    return i < std::size(kNames) ? kNames[i] : std::string_view("unknown");
}

void register_kernel(const KernelRegistration &entry) {
    if (const char *defect = defect_of(entry)) {
        std::fprintf(stderr, "pfng_bench: refusing kernel \"%.*s\": %s\n", static_cast<int>(entry.id.size()),
                     entry.id.data(), defect);
        std::abort();
    }
    Catalogue &c = catalogue();
    c.index_of.emplace(std::string(entry.id), c.entries.size());
    c.entries.push_back(entry);
}

std::span<const KernelRegistration> registered_kernels() { return catalogue().entries; }

const KernelRegistration *find_kernel(std::string_view id) {
    const Catalogue &c = catalogue();
    const auto hit = c.index_of.find(std::string(id));
    return hit == c.index_of.end() ? nullptr : &c.entries[hit->second];
}

}  // namespace pfng::bench

#include "registry.h"

#include <cstdio>
#include <cstdlib>

namespace pfng::bench {

namespace {

std::vector<KernelRegistration> &table() {
    static std::vector<KernelRegistration> kernels;
    return kernels;
}

[[noreturn]] void reject(std::string_view why, std::string_view id) {
    std::fprintf(stderr, "kernel registration error for '%.*s': %.*s\n", (int)id.size(), id.data(), (int)why.size(),
                 why.data());
    std::abort();
}

}  // namespace

std::string_view quantization_name(QuantizationType type) {
    switch (type) {
    case QuantizationType::WeightQ4_0ActivationQ8_0: return "WeightQ4_0ActivationQ8_0";
    case QuantizationType::WeightQ4_KActivationQ8_K: return "WeightQ4_KActivationQ8_K";
    case QuantizationType::WeightIQ2_XXSActivationQ8_K: return "WeightIQ2_XXSActivationQ8_K";
    default: return "unknown";
    }
}

void register_kernel(const KernelRegistration &r) {
    if (r.id.empty()) reject("empty id", r.id);
    if (r.name.empty()) reject("empty name", r.id);
    const KernelCallbacks &c = r.callbacks;
    if (!c.peak_performance || !c.validate || !c.prepare || !c.reset || !c.run || !c.export_output || !c.checksum ||
        !c.destroy)
        reject("missing required callback", r.id);
    if ((size_t)r.quantization >= (size_t)QuantizationType::Count) reject("unknown quantization type", r.id);
    if (find_kernel(r.id)) reject("duplicate id", r.id);
    table().push_back(r);
}

std::span<const KernelRegistration> registered_kernels() { return table(); }

const KernelRegistration *find_kernel(std::string_view id) {
    for (const KernelRegistration &k : table())
        if (k.id == id) return &k;
    return nullptr;
}

}  // namespace pfng::bench

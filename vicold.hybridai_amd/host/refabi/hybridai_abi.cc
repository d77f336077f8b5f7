// hybridai_abi.cc -- registries for the standalone build of the backend ABI
// (in a reference build these come from src/backends/backend_registry.cc
// and src/ops/registry.cc instead, and this file is not compiled).
#include "hybridai_abi.h"

#ifndef HAI_WITH_REFERENCE_TREE

namespace hybridai {

BackendRegistry& BackendRegistry::instance() {
    static BackendRegistry registry;
    return registry;
}

void BackendRegistry::register_backend(std::string_view name, BackendFactory factory) {
    std::lock_guard<std::mutex> lock(mutex_);
    const std::string key(name);
    factories_[key] = std::move(factory);
    // a re-registered name drops the instances made by the old factory
    const std::string prefix = key + ":";
    for (auto it = backends_.begin(); it != backends_.end();) {
        if (it->first.compare(0, prefix.size(), prefix) == 0) it = backends_.erase(it);
        else ++it;
    }
}

std::unique_ptr<Backend> BackendRegistry::create_backend(const Device& device) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (device.backend().empty()) return nullptr;
    auto it = factories_.find(device.backend());
    return it == factories_.end() ? nullptr : it->second(device);
}

std::shared_ptr<Backend> BackendRegistry::get_backend(const Device& device) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (device.backend().empty()) return nullptr;
    const std::string key = device.backend() + ":" + std::to_string(device.id()) + ":" +
                            std::to_string(static_cast<unsigned>(device.type()));
    if (auto hit = backends_.find(key); hit != backends_.end()) return hit->second;
    auto it = factories_.find(device.backend());
    if (it == factories_.end()) return nullptr;
    std::shared_ptr<Backend> made = it->second(device);
    if (made) backends_.emplace(key, made);
    return made;
}

bool BackendRegistry::has_backend(std::string_view name) const {
    std::lock_guard<std::mutex> lock(mutex_);
    return factories_.count(std::string(name)) != 0;
}

std::vector<std::string> BackendRegistry::backend_names() const {
    std::lock_guard<std::mutex> lock(mutex_);
    std::vector<std::string> names;
    for (const auto& kv : factories_) names.push_back(kv.first);
    return names;
}

namespace ops {

KernelRegistry& KernelRegistry::instance() {
    static KernelRegistry registry;
    return registry;
}

bool KernelRegistry::register_kernel(const KernelKey& key, KernelFn kernel, bool overwrite) {
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = kernels_.find(key);
    if (it != kernels_.end() && !overwrite) return false;
    kernels_[key] = std::move(kernel);
    return true;
}

KernelFn KernelRegistry::find_kernel(const KernelKey& key) const {
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = kernels_.find(key);
    return it == kernels_.end() ? KernelFn{} : it->second;
}

bool KernelRegistry::has_kernel(const KernelKey& key) const {
    std::lock_guard<std::mutex> lock(mutex_);
    return kernels_.count(key) != 0;
}

bool KernelRegistry::unregister_kernel(const KernelKey& key) {
    std::lock_guard<std::mutex> lock(mutex_);
    return kernels_.erase(key) != 0;
}

size_t KernelRegistry::kernel_count() const {
    std::lock_guard<std::mutex> lock(mutex_);
    return kernels_.size();
}

}  // namespace ops
}  // namespace hybridai

#endif  // HAI_WITH_REFERENCE_TREE

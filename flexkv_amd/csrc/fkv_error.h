// Internal: the calling thread's last error message, shared by the library's
// translation units and returned by fkv_last_error(), and the host block ids
// its last failed transfer left to copies given up on, returned by
// fkv_last_unsafe_host_blocks().
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace fkv_detail {
__attribute__((visibility("hidden"))) std::string& last_error();
__attribute__((visibility("hidden"))) std::vector<int64_t>& last_unsafe_host_blocks();
}  // namespace fkv_detail

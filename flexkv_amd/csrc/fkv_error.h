// Internal: the calling thread's last error message, shared by the library's
// translation units and returned by fkv_last_error().
#pragma once
#include <string>

namespace fkv_detail {
__attribute__((visibility("hidden"))) std::string& last_error();
}  // namespace fkv_detail

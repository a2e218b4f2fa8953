#pragma once
// Helpers shared by the host side of libq35.so: error reporting and the conversion between
// the C-ABI dims struct and ModelConfig.
#include <string>

#include "../../include/q35.h"
#include "model_config.h"

namespace q35 {

// Records a message for q35_last_error() and returns `code`.
q35_status fail(q35_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char* last_error_cstr();

void dims_from_config(const ModelConfig& c, q35_dims* d);

// Counts a device allocation the library made (reported by q35_device_alloc_count).
void count_device_alloc();
ModelConfig config_from_dims(const q35_dims& d);

}  // namespace q35

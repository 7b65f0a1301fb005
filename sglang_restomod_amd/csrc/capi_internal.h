// Internal helpers shared by the C-ABI entry points.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/mi355x_attn.h"

// Record a formatted message as this thread's last error and return `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

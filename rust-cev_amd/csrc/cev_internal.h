// Internal helpers shared by the host code and the launchers.
#pragma once
#include <stdarg.h>
#include <stdint.h>

#include "../../include/cev_hip.h"

// Records a formatted thread-local message for cev_last_error() and returns
// `code`, so call sites read `return cev_fail(CEV_ERR_INVALID, "...", ...)`.
int32_t cev_fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void cev_clear_error();

#define CEV_CHECK_ARG(cond, ...)                      \
  do {                                                \
    if (!(cond)) return cev_fail(CEV_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// Validates an attention descriptor (dtype, shapes, strides, scale); the
// planner runs it on every plan build and the launcher on every launch.
int32_t cev_check_attn_desc(const cev_attn_desc* d);

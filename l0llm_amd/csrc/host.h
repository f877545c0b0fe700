// Internal host helpers shared by the matrix and model code.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

namespace l0h {
uint16_t host_f32_to_f16(float f);
float host_f16_to_f32(uint16_t h);
uint16_t host_f32_to_bf16(float f);
void quantize_rows(const float* w, int n, int k, int8_t* q, uint16_t* s);
}  // namespace l0h

// Fixed per-device scratch of ifr_matmul_quant_noalloc (csrc/noalloc.hip).
#pragma once
#include <hip/hip_runtime_api.h>
#include <stdint.h>

// Bytes of the array: the quantized input of the largest GEMV the integer
// path takes (3 * 18432 + 18432 / 2 = 64512 bytes), rounded up.
#define IFR_NOALLOC_SCRATCH_BYTES 65536

// Device address of `device`'s array, looked up once per device with that
// device current (hipGetSymbolAddress).
hipError_t ifr_noalloc_init(int device, void **ptr);

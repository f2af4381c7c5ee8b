// Host functions that one source file of the library calls in another.
#pragma once

#include "h3_common.hpp"

namespace h3 {

// The argument checks of launch_h3_quantize_fp8_per_head(stream, x, x8,
// descale) alone: 0 when the call would be accepted, kInvalid otherwise. No
// HIP call. (h3_attention_fp8.hip)
int check_quantize_fp8_per_head(const NineToothedTensor &x, const NineToothedTensor &x8,
                                const NineToothedTensor &descale);

// The number of CUs of device `dev`, looked up once per device; 0 when the
// lookup fails. (h3_attention.hip)
int device_cus(int dev);

// The same for the device `stream` belongs to. (h3_attention.hip)
int stream_device_cus(hipStream_t stream);

}  // namespace h3

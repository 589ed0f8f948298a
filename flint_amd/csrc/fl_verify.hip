// Speculative verify (M = k+1 tokens per pass) and the M<=16 int4 GEMM.
#include "fl_common.h"

extern "C" {

int fl_verify(const fl_weights*, fl_state*, const int32_t*, int32_t, const int32_t*,
              const uint8_t*, int32_t, int32_t*, float*, uint16_t*, void*) {
  return FL_E_ARG;
}

}  // extern "C"

// Link stub for the CPU sanitizer build of the loader: the device dequant is
// never reached by the fuzz driver (it loads nothing to a device).
#include "nf4stream.h"
#include <cstdlib>
extern "C" int32_t nf4s_dequant_f16(const nf4s_tensor *, int64_t, uint16_t *, void *) { abort(); }

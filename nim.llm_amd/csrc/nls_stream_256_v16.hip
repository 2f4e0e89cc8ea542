// stream_kernel for 256-thread workgroups with 16-byte loads (see nls_stream_inst.h).
#include "nls_stream_inst.h"

NLS_INSTANTIATE_STREAM(256, true)

// stream_kernel for 512-thread workgroups with 16-byte loads (see nls_stream_inst.h).
#include "nls_stream_inst.h"

NLS_INSTANTIATE_STREAM(512, true)

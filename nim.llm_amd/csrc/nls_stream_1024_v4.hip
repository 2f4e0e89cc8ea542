// stream_kernel for 1024-thread workgroups with 4-byte loads (see nls_stream_inst.h).
#include "nls_stream_inst.h"

NLS_INSTANTIATE_STREAM(1024, false)

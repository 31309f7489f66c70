// The control step with each world's working set in a slab of the caller's `workspace` array
// (device memory) instead of LDS: the same source compiled with global-memory working-set
// pointers into namespace mx_slab.  Used for models whose working set exceeds the LDS of one
// workgroup (the 20-object dense-clutter scenes) and on request (MX_FLAG_WORKSPACE).
#define MX_SLAB 1
#define MX_NS mx_slab
#include "mx_step.hip"

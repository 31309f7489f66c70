// The FP64 route of the control step: the same source in namespace mx_f64 with the physics
// working type `real` = double (positions, frames, inertias, mass matrices and their inverses,
// collision geometry, constraint rows, forces, the Newton solve), the working set in LDS.  The
// model image stays 32-bit (the model arena is FP32), the world state enters and leaves through
// the FP32 fields of MxData, and the controller is the FP64 OSC of every build.  Selected by
// MX_FLAG_FP64 for models whose FP64 working set fits the workgroup's LDS (mx_lds_bytes_fp64).
#define MX_F64 1
#define MX_NS mx_f64
#include "mx_step.hip"

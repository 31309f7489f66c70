// The workspace-route control step with four island-sweep entries per lane (see kOwn in
// mx_step.hip): the same source in namespace mx_slab4, chosen at launch for models whose
// contact-free island blocks are small.  Its slabs are never larger than mx_slab's, whose size the
// workspace is checked against.
#define MX_SLAB 1
#define MX_NS mx_slab4
#define MX_OWN 4
#include "mx_step.hip"

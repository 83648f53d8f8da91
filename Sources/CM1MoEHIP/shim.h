/* Umbrella header of the CM1MoEHIP module.  The declarations live in the
 * library's own header (include/m1moe_hip.h of the libm1moe_hip source
 * tree); the include path to it comes from the dependent target's
 * `-Xcc -I<root>/include` (Package.swift.fragment), so this directory holds
 * no copy that could drift from the library it links. */
#ifndef CM1MOEHIP_SHIM_H
#define CM1MOEHIP_SHIM_H
#include <m1moe_hip.h>
#endif

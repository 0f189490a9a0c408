/*
 * gsx_hip_type.h - the declarations a gsx tree adds to make the MI355X backend a backend type
 * of its own instead of a tenant of the CUDA slot. TEST HARNESS: force-included (-include)
 * into the gsx core's gsx-backend.c, into ref_driver.c and into a second build of the plugin
 * for oracle/_ref/libgsxref_hiptype.so; the reference sources themselves stay as they lie.
 *
 * A gsx tree that takes the backend for good makes the same three additions in its own files:
 *   - GSX_BACKEND_TYPE_HIP = 3 as an enumerator of gsx_backend_type
 *     (gsx/include/gsx/gsx-backend.h:8-12);
 *   - the bootstrap declaration under GSX_HAS_HIP beside the CUDA one (gsx/src/gsx-impl.h:676-681);
 *   - GSX_HAS_HIP defaulting to 0 beside GSX_HAS_CUDA (gsx/src/gsx-impl.h:11-17).
 * hip_backend_type.sed makes the two additions to gsx-backend.c (the type check and the
 * bootstrap call). Here the type is a constant of the enum's type, which compiles to the same
 * code as the enumerator.
 */
#ifndef GSX_HIP_TYPE_H
#define GSX_HIP_TYPE_H

#include "gsx-impl.h"

#ifndef GSX_HAS_HIP
#define GSX_HAS_HIP 1
#endif

#define GSX_BACKEND_TYPE_HIP ((gsx_backend_type)3)

GSX_EXTERN_C_BEGIN
gsx_error gsx_hip_backend_provider_bootstrap(gsx_builtin_registry_state *registry);
GSX_EXTERN_C_END

#endif /* GSX_HIP_TYPE_H */

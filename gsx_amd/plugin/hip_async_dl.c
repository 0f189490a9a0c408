/*
 * hip_async_dl.c - the gsx_async_dl_i entry of the gsx HIP backend (gsx/src/gsx-impl.h:524-529).
 * The backend reports supports_async_prefetch = false, so gsx's dataloader stages samples on the
 * caller's thread (gsx/src/gsx-data.c:538-589) and never asks for an async loader.
 */
#include "hip_backend.h"

gsx_error gsx_hip_plugin_create_async_dl(gsx_backend_t backend, const gsx_async_dl_desc *desc, gsx_async_dl_t *out)
{
    (void)backend;
    (void)desc;
    if(out != NULL) {
        *out = NULL;
    }
    return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip backend has no async dataloader");
}

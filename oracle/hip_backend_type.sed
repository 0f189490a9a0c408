# The two additions to gsx/src/gsx-backend.c that make HIP a backend type of its own, applied
# to the source as it lies while it streams into the compiler (no copy is written):
#   1. the registry's type check (gsx-backend.c:184-194) accepts GSX_BACKEND_TYPE_HIP;
#   2. gsx_backend_registry_init (gsx-backend.c:215-251) calls the HIP provider's bootstrap after
#      the CUDA one, with the same NOT_SUPPORTED rule (no device: init still succeeds).
# GSX_BACKEND_TYPE_HIP, GSX_HAS_HIP and the bootstrap's declaration come from gsx_hip_type.h.
/^    case GSX_BACKEND_TYPE_METAL:$/a\
    case GSX_BACKEND_TYPE_HIP:
/^#if GSX_HAS_METAL$/i\
#if GSX_HAS_HIP\
    error = gsx_hip_backend_provider_bootstrap(registry);\
    if(error.code == GSX_ERROR_NOT_SUPPORTED) {\
        GSX_LOG_WARN("backend: hip provider not available\\n");\
        error = gsx_make_error(GSX_ERROR_SUCCESS, NULL);\
    }\
    if(!gsx_error_is_success(error)) {\
        gsx_builtin_registry_reset(registry);\
        return error;\
    }\
#endif

/*
 * ggml_hip_reg.h -- the dlopen entry points of libggml-hip.so, the loadable
 * backend module that puts this library behind llama.rust's dynamic backend
 * registry (ggml_backend_load / ggml_backend_load_best,
 * crates/ggml/src/backend.rs:1345-1420, :1587-1660).
 *
 * The loader dlopens the module, calls ggml_backend_score() when it is
 * exported (0 = "not supported on this system"), then ggml_backend_init(),
 * and accepts the returned registry object only if api_version == 2
 * (GGML_BACKEND_API_VERSION, backend.rs:44).  Through the object it reads
 * the backend name, the device count, each device's name, description,
 * memory and type, and -- by name, with get_proc_address -- the compute
 * entry points of ghip.h.  The struct layouts below are the ones the loader
 * reads (GgmlBackendRegI / GgmlBackendReg / GgmlBackendDeviceI /
 * GgmlBackendDevice, crates/ggml/src/sysffi.rs:131-171, field order is the
 * ABI).
 */
#ifndef GGML_HIP_REG_H
#define GGML_HIP_REG_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_HIP_BACKEND_API_VERSION 2

typedef struct ggml_hip_backend_reg ggml_hip_backend_reg;
typedef struct ggml_hip_backend_device ggml_hip_backend_device;

/* struct ggml_backend_reg_i (sysffi.rs:131-138) */
typedef struct ggml_hip_backend_reg_i {
    const char *(*get_name)(const ggml_hip_backend_reg *reg);
    size_t (*get_device_count)(const ggml_hip_backend_reg *reg);
    ggml_hip_backend_device *(*get_device)(const ggml_hip_backend_reg *reg, size_t index);
    /* "ghip_init", "ghip_mul_mat", ... -> the ghip.h function of that name,
     * NULL for any other name */
    void *(*get_proc_address)(const ggml_hip_backend_reg *reg, const char *name);
} ggml_hip_backend_reg_i;

/* struct ggml_backend_reg (sysffi.rs:140-147) */
struct ggml_hip_backend_reg {
    int api_version; /* GGML_HIP_BACKEND_API_VERSION */
    ggml_hip_backend_reg_i iface;
    void *context;
};

/* struct ggml_backend_device_i (sysffi.rs:149-157) */
typedef struct ggml_hip_backend_device_i {
    const char *(*get_name)(const ggml_hip_backend_device *dev);        /* "HIP0", "HIP1", ... */
    const char *(*get_description)(const ggml_hip_backend_device *dev); /* the HIP device name */
    void (*get_memory)(const ggml_hip_backend_device *dev, size_t *free, size_t *total);
    int (*get_type)(const ggml_hip_backend_device *dev); /* 1 = GGML_BACKEND_DEVICE_TYPE_GPU */
} ggml_hip_backend_device_i;

/* struct ggml_backend_device (sysffi.rs:159-171); context holds the HIP
 * device ordinal (intptr_t) to pass to ghip_init */
struct ggml_hip_backend_device {
    ggml_hip_backend_device_i iface;
    const ggml_hip_backend_reg *reg;
    void *context;
};

/* ggml_backend_score_t (sysffi.rs:120-121): 0 when no gfx950 device is
 * visible, otherwise a positive score (higher = preferred by
 * ggml_backend_load_best, backend.rs:1587-1660). */
int ggml_backend_score(void);

/* ggml_backend_init_t (sysffi.rs:118-119): the module's registry object
 * (static, never freed); its device list is fixed at the first call. */
ggml_hip_backend_reg *ggml_backend_init(void);

#ifdef __cplusplus
}
#endif
#endif

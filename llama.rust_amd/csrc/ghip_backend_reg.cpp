// libggml-hip.so: the dlopen module of this backend for llama.rust's dynamic
// backend registry (ggml_backend_load, crates/ggml/src/backend.rs:1354-1420).
// It exports ggml_backend_score / ggml_backend_init and hands out the
// compute entry points of libghip.so by name through get_proc_address.
// HIP is only asked for device counts, names and memory; compute goes
// through ghip_init and the ghip_* calls.
#include "ggml_hip_reg.h"
#include "ghip.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

namespace {

struct DeviceSlot {
    ggml_hip_backend_device dev;
    char name[16];
    char description[256];
};

std::once_flag g_once;
std::vector<DeviceSlot> *g_devices = nullptr;  // fixed after the first ggml_backend_init
ggml_hip_backend_reg g_reg;

// gfx950 devices only: the code objects next to libghip.so are built for it
bool is_gfx950(int ordinal, hipDeviceProp_t *prop) {
    if (hipGetDeviceProperties(prop, ordinal) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return std::strncmp(prop->gcnArchName, "gfx950", 6) == 0;
}

int visible_devices() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();  // no HIP device: not an error of the caller's next call
        return 0;
    }
    return n;
}

const char *dev_name(const ggml_hip_backend_device *d) {
    return reinterpret_cast<const DeviceSlot *>(d)->name;
}

const char *dev_description(const ggml_hip_backend_device *d) {
    return reinterpret_cast<const DeviceSlot *>(d)->description;
}

// hipMemGetInfo reports the current device: switch to this one and back
void dev_memory(const ggml_hip_backend_device *d, size_t *free_b, size_t *total_b) {
    *free_b = 0;
    *total_b = 0;
    const int ordinal = (int)(intptr_t)d->context;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (hipSetDevice(ordinal) == hipSuccess) {
        if (hipMemGetInfo(free_b, total_b) != hipSuccess) {
            *free_b = 0;
            *total_b = 0;
        }
    }
    (void)hipGetLastError();
    if (prev >= 0) (void)hipSetDevice(prev);
}

int dev_type(const ggml_hip_backend_device *) { return 1; }  // GGML_BACKEND_DEVICE_TYPE_GPU

const char *reg_name(const ggml_hip_backend_reg *) { return "HIP"; }

size_t reg_device_count(const ggml_hip_backend_reg *) { return g_devices ? g_devices->size() : 0; }

ggml_hip_backend_device *reg_device(const ggml_hip_backend_reg *, size_t index) {
    if (!g_devices || index >= g_devices->size()) return nullptr;
    return &(*g_devices)[index].dev;
}

struct Proc {
    const char *name;
    void *fn;
};

void *reg_proc_address(const ggml_hip_backend_reg *, const char *name) {
    static const Proc procs[] = {
        {"ghip_init", (void *)&ghip_init},
        {"ghip_init_dry_run", (void *)&ghip_init_dry_run},
        {"ghip_free", (void *)&ghip_free},
        {"ghip_last_error", (void *)&ghip_last_error},
        {"ghip_synchronize", (void *)&ghip_synchronize},
        {"ghip_supports_op", (void *)&ghip_supports_op},
        {"ghip_mul_mat", (void *)&ghip_mul_mat},
        {"ghip_mul_mat_noalloc", (void *)&ghip_mul_mat_noalloc},
        {"ghip_mul_mat_subsums", (void *)&ghip_mul_mat_subsums},
        {"ghip_mul_mat_act", (void *)&ghip_mul_mat_act},
        {"ghip_mul_mat_id", (void *)&ghip_mul_mat_id},
        {"ghip_mul_mat_id_subsums", (void *)&ghip_mul_mat_id_subsums},
        {"ghip_flash_attn_ext", (void *)&ghip_flash_attn_ext},
        {"ghip_quantize_chunk", (void *)&ghip_quantize_chunk},
        {"ghip_graph_compute", (void *)&ghip_graph_compute},
        {"ghip_set_workspace", (void *)&ghip_set_workspace},
        {"ghip_workspace_size", (void *)&ghip_workspace_size},
        {"ghip_weight_register", (void *)&ghip_weight_register},
        {"ghip_weight_unregister", (void *)&ghip_weight_unregister},
        {"ghip_weight_cache_stats", (void *)&ghip_weight_cache_stats},
        {"ghip_gguf_alignment", (void *)&ghip_gguf_alignment},
        {"ghip_gguf_arr_n", (void *)&ghip_gguf_arr_n},
        {"ghip_gguf_arr_type", (void *)&ghip_gguf_arr_type},
        {"ghip_gguf_close", (void *)&ghip_gguf_close},
        {"ghip_gguf_data_offset", (void *)&ghip_gguf_data_offset},
        {"ghip_gguf_find_key", (void *)&ghip_gguf_find_key},
        {"ghip_gguf_find_tensor", (void *)&ghip_gguf_find_tensor},
        {"ghip_gguf_get_bool", (void *)&ghip_gguf_get_bool},
        {"ghip_gguf_get_f32", (void *)&ghip_gguf_get_f32},
        {"ghip_gguf_get_f64", (void *)&ghip_gguf_get_f64},
        {"ghip_gguf_get_i64", (void *)&ghip_gguf_get_i64},
        {"ghip_gguf_get_str", (void *)&ghip_gguf_get_str},
        {"ghip_gguf_get_u16", (void *)&ghip_gguf_get_u16},
        {"ghip_gguf_get_u32", (void *)&ghip_gguf_get_u32},
        {"ghip_gguf_key", (void *)&ghip_gguf_key},
        {"ghip_gguf_kv_type", (void *)&ghip_gguf_kv_type},
        {"ghip_gguf_n_kv", (void *)&ghip_gguf_n_kv},
        {"ghip_gguf_n_parts", (void *)&ghip_gguf_n_parts},
        {"ghip_gguf_n_tensors", (void *)&ghip_gguf_n_tensors},
        {"ghip_gguf_open", (void *)&ghip_gguf_open},
        {"ghip_gguf_tensor", (void *)&ghip_gguf_tensor},
        {"ghip_gguf_tensor_data", (void *)&ghip_gguf_tensor_data},
        {"ghip_gguf_upload", (void *)&ghip_gguf_upload},
        {"ghip_gguf_version", (void *)&ghip_gguf_version},
    };
    if (!name) return nullptr;
    for (const Proc &p : procs)
        if (std::strcmp(p.name, name) == 0) return p.fn;
    return nullptr;
}

void build_registry() {
    g_reg.api_version = GGML_HIP_BACKEND_API_VERSION;
    g_reg.iface.get_name = reg_name;
    g_reg.iface.get_device_count = reg_device_count;
    g_reg.iface.get_device = reg_device;
    g_reg.iface.get_proc_address = reg_proc_address;
    g_reg.context = nullptr;
    auto *devs = new std::vector<DeviceSlot>();
    const int n = visible_devices();
    devs->reserve(n > 0 ? (size_t)n : 0);  // no reallocation below: device pointers stay valid
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t prop;
        if (!is_gfx950(i, &prop)) continue;
        DeviceSlot s{};
        std::snprintf(s.name, sizeof(s.name), "HIP%zu", devs->size());
        std::snprintf(s.description, sizeof(s.description), "%s", prop.name);
        s.dev.iface.get_name = dev_name;
        s.dev.iface.get_description = dev_description;
        s.dev.iface.get_memory = dev_memory;
        s.dev.iface.get_type = dev_type;
        s.dev.reg = &g_reg;
        s.dev.context = (void *)(intptr_t)i;
        devs->push_back(s);
    }
    g_devices = devs;
}

}  // namespace

extern "C" {

int ggml_backend_score(void) {
    const int n = visible_devices();
    int found = 0;
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t prop;
        if (is_gfx950(i, &prop)) found++;
    }
    return found ? 100 : 0;
}

ggml_hip_backend_reg *ggml_backend_init(void) {
    std::call_once(g_once, build_registry);
    return &g_reg;
}

}  // extern "C"

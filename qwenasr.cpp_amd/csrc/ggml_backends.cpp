// ggml-backends.h drop-in: device selection for the MI355X build.
//
// Same string parsing, names and environment toggles as the reference (src/ggml-backends.cpp:21-100):
// "auto", "cpu", "gpu" and the alias "cuda", case-insensitive.  Backend-set initialisation
// (reference 127-165) differs on purpose: the primary backend is HIP device 0 and there is no CPU
// fallback backend, so a request that the reference would have served on the CPU ("cpu", or "auto"
// without a GPU) fails with a message instead of running a different implementation.
#include "ggml-backends.h"

#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <string>

#include "qwenasr_amd.h"

struct ggml_backend {
    int device = 0;
    std::string name;
};

namespace {

void set_error(std::string * error, const std::string & message) {
    if (error) *error = message;
}

std::string lower_ascii(std::string value) {
    std::transform(value.begin(), value.end(), value.begin(),
                   [](unsigned char ch) { return static_cast<char>(std::tolower(ch)); });
    return value;
}

bool env_flag(const char * name, bool default_value) {
    const char * value = std::getenv(name);
    if (!value || value[0] == '\0') return default_value;
    const std::string v = lower_ascii(value);
    return v != "0" && v != "false" && v != "off" && v != "no";
}

}  // namespace

QwenAsrGgmlDevice qwenasr_ggml_device_auto() { return QwenAsrGgmlDevice::Auto; }
QwenAsrGgmlDevice qwenasr_ggml_device_cpu() { return QwenAsrGgmlDevice::Cpu; }
QwenAsrGgmlDevice qwenasr_ggml_device_gpu() { return QwenAsrGgmlDevice::Gpu; }

bool qwenasr_ggml_device_from_string(const std::string & value, QwenAsrGgmlDevice * out, std::string * error) {
    if (!out) {
        set_error(error, "qwenasr_ggml_device_from_string: out is null");
        return false;
    }
    const std::string v = lower_ascii(value);
    if (v == "auto") {
        *out = QwenAsrGgmlDevice::Auto;
        return true;
    }
    if (v == "cpu") {
        *out = QwenAsrGgmlDevice::Cpu;
        return true;
    }
    if (v == "gpu" || v == "cuda") {
        *out = QwenAsrGgmlDevice::Gpu;
        return true;
    }
    set_error(error, "GGML device must be auto, cpu, gpu, or cuda");
    return false;
}

const char * qwenasr_ggml_device_name(QwenAsrGgmlDevice device) {
    switch (device) {
        case QwenAsrGgmlDevice::Auto: return "auto";
        case QwenAsrGgmlDevice::Cpu: return "cpu";
        case QwenAsrGgmlDevice::Gpu: return "gpu";
    }
    return "unknown";
}

bool qwenasr_ggml_flash_attn_enabled() { return env_flag("QWENASR_GGML_FLASH_ATTN", false); }

bool qwenasr_ggml_combined_audio_enabled() { return env_flag("QWENASR_GGML_COMBINED_AUDIO", true); }

bool qwenasr_ggml_backend_set_init(QwenAsrGgmlDevice device, int n_threads, QwenAsrGgmlBackendSet * out,
                                   std::string * error) {
    (void)n_threads;
    if (!out) {
        set_error(error, "qwenasr_ggml_backend_set_init: out is null");
        return false;
    }
    out->primary = nullptr;
    out->fallback = nullptr;
    if (device == QwenAsrGgmlDevice::Cpu) {
        set_error(error, "this build runs the text decoder on HIP device 0 only; --device cpu is not available");
        return false;
    }
    if (qa_device_count() <= 0) {
        set_error(error, device == QwenAsrGgmlDevice::Gpu
                             ? "failed to initialize requested GPU backend; no HIP device is visible"
                             : "no HIP device is visible and this build has no CPU fallback backend");
        return false;
    }
    char arch[64] = {0};
    qa_device_arch(arch, sizeof(arch));
    ggml_backend * b = new ggml_backend();
    b->device = 0;
    b->name = std::string("HIP0 (") + arch + ")";
    out->primary = b;
    return true;
}

void qwenasr_ggml_backend_set_free(QwenAsrGgmlBackendSet * backends) {
    if (!backends) return;
    delete backends->fallback;
    delete backends->primary;
    backends->fallback = nullptr;
    backends->primary = nullptr;
}

int qwenasr_ggml_backend_set_count(const QwenAsrGgmlBackendSet & backends) {
    return (backends.primary ? 1 : 0) + (backends.fallback ? 1 : 0);
}

void qwenasr_ggml_backend_set_array(const QwenAsrGgmlBackendSet & backends, ggml_backend_t out[2]) {
    out[0] = backends.primary;
    out[1] = backends.fallback;
}

const char * qwenasr_ggml_backend_set_primary_name(const QwenAsrGgmlBackendSet & backends) {
    return backends.primary ? backends.primary->name.c_str() : "none";
}

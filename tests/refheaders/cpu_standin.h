// cpu_standin.h - a CPU device for the reference's backend_init
// (src/backend.h:37-50, :135-146), which exits without one, for the drivers
// that run the reference's model code on the MI355X backend (test
// infrastructure).  It runs nothing: supports_op is false for every op, so
// the scheduler places every graph on the MI355X backend.  Its buffers are
// plain host memory.  Also the file helpers the drivers share.
#pragma once

#include "ggml-backend-impl.h"
#include "ggml-backend.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <fstream>
#include <string>
#include <vector>

namespace refdrv {

struct host_buf {
    std::vector<uint8_t> bytes;
};

void hb_free(ggml_backend_buffer_t b) {
    delete (host_buf *) b->context;
}
void * hb_base(ggml_backend_buffer_t b) {
    return ((host_buf *) b->context)->bytes.data();
}
void hb_memset(ggml_backend_buffer_t, ggml_tensor * t, uint8_t v, size_t off, size_t n) {
    memset((char *) t->data + off, v, n);
}
void hb_set(ggml_backend_buffer_t, ggml_tensor * t, const void * d, size_t off, size_t n) {
    memcpy((char *) t->data + off, d, n);
}
void hb_get(ggml_backend_buffer_t, const ggml_tensor * t, void * d, size_t off, size_t n) {
    memcpy(d, (const char *) t->data + off, n);
}
void hb_clear(ggml_backend_buffer_t b, uint8_t v) {
    std::vector<uint8_t> & x = ((host_buf *) b->context)->bytes;
    memset(x.data(), v, x.size());
}
const ggml_backend_buffer_i k_hb_iface = { hb_free, hb_base, nullptr, hb_memset, hb_set, hb_get, nullptr, hb_clear,
                                           nullptr };

const char * hbt_name(ggml_backend_buffer_type_t) {
    return "CPU";
}
ggml_backend_buffer_t hbt_alloc(ggml_backend_buffer_type_t t, size_t size) {
    auto * h = new host_buf();
    h->bytes.resize(size + 64);
    return ggml_backend_buffer_init(t, k_hb_iface, h, size);
}
size_t hbt_align(ggml_backend_buffer_type_t) {
    return 64;
}
bool hbt_is_host(ggml_backend_buffer_type_t) {
    return true;
}

const char * cb_name(ggml_backend_t) {
    return "CPU";
}
void cb_free(ggml_backend_t b) {
    delete b;
}
void cb_sync(ggml_backend_t) {}
ggml_status cb_compute(ggml_backend_t, ggml_cgraph *) {
    fprintf(stderr, "[driver] the CPU stand-in was asked to compute a graph\n");
    return GGML_STATUS_FAILED;
}
ggml_guid k_cpu_guid = { { 'c', 'p', 'u', '-', 's', 't', 'a', 'n', 'd', '-', 'i', 'n', 0, 0, 0, 1 } };
const ggml_backend_i k_cb_iface = { cb_name, cb_free, nullptr, nullptr, nullptr, cb_sync, nullptr,
                                    nullptr, nullptr, nullptr, cb_compute, nullptr, nullptr, nullptr };

ggml_backend_buffer_type g_host_buft;
ggml_backend_device      g_cpu_dev;
ggml_backend_reg         g_cpu_reg;

const char * cd_name(ggml_backend_dev_t) {
    return "CPU";
}
const char * cd_desc(ggml_backend_dev_t) {
    return "host stand-in (runs no ops)";
}
void cd_mem(ggml_backend_dev_t, size_t * f, size_t * t) {
    *f = 0;
    *t = 0;
}
enum ggml_backend_dev_type cd_type(ggml_backend_dev_t) {
    return GGML_BACKEND_DEVICE_TYPE_CPU;
}
void cd_props(ggml_backend_dev_t d, ggml_backend_dev_props * p) {
    p->name        = cd_name(d);
    p->description = cd_desc(d);
    p->memory_free = p->memory_total = 0;
    p->type        = GGML_BACKEND_DEVICE_TYPE_CPU;
    p->device_id   = nullptr;
    p->caps        = { false, false, false, false };
}
ggml_backend_t cd_init(ggml_backend_dev_t d, const char *) {
    return new ggml_backend{ &k_cpu_guid, k_cb_iface, d, nullptr };
}
ggml_backend_buffer_type_t cd_buft(ggml_backend_dev_t) {
    return &g_host_buft;
}
bool cd_supports_op(ggml_backend_dev_t, const ggml_tensor *) {
    return false;
}
bool cd_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t t) {
    return ggml_backend_buft_is_host(t);
}
const ggml_backend_device_i k_cd_iface = { cd_name, cd_desc, cd_mem,         cd_type,          cd_props, cd_init,
                                           cd_buft, nullptr, nullptr,        cd_supports_op,   cd_supports_buft,
                                           nullptr, nullptr, nullptr,        nullptr };

const char * cr_name(ggml_backend_reg_t) {
    return "CPU";
}
size_t cr_count(ggml_backend_reg_t) {
    return 1;
}
ggml_backend_dev_t cr_dev(ggml_backend_reg_t, size_t i) {
    return i == 0 ? &g_cpu_dev : nullptr;
}
void set_n_threads(ggml_backend_t, int) {}
void * cr_proc(ggml_backend_reg_t, const char * name) {
    return strcmp(name, "ggml_backend_set_n_threads") == 0 ? (void *) set_n_threads : nullptr;
}
const ggml_backend_reg_i k_cr_iface = { cr_name, cr_count, cr_dev, cr_proc };

void register_cpu_standin() {
    g_host_buft = { { hbt_name, hbt_alloc, hbt_align, nullptr, nullptr, hbt_is_host }, &g_cpu_dev, nullptr };
    g_cpu_reg   = { GGML_BACKEND_API_VERSION, k_cr_iface, nullptr };
    g_cpu_dev   = { k_cd_iface, &g_cpu_reg, nullptr };
    ggml_backend_register(&g_cpu_reg);
}

template <typename T> std::vector<T> read_vec(const std::string & path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) {
        fprintf(stderr, "[driver] cannot read %s\n", path.c_str());
        exit(2);
    }
    const size_t n = (size_t) f.tellg();
    f.seekg(0);
    std::vector<T> v(n / sizeof(T));
    f.read((char *) v.data(), (std::streamsize) (v.size() * sizeof(T)));
    return v;
}

void write_bytes(const std::string & path, const void * p, size_t n) {
    std::ofstream f(path, std::ios::binary);
    f.write((const char *) p, (std::streamsize) n);
    if (!f) {
        fprintf(stderr, "[driver] cannot write %s\n", path.c_str());
        exit(2);
    }
}

}  // namespace refdrv

// dit_driver.cpp - runs the reference's flow-matching DiT (src/dit.h with
// src/gguf-weights.h, src/weight-ctx.h, src/backend.h), compiled unchanged
// from the reference tree, on the MI355X ggml backend through this build's
// ggml API layer.  Test infrastructure: tests/test_gpu_refheaders.py writes
// the GGUF and the inputs, runs this program and checks what it writes.
//
//   dit_driver <dit.gguf> <io_dir> <T> <B> <t> <n_runs>
//
// io_dir/xt.bin (f32 B x [T, 128] time-major blocks) and io_dir/cond.bin (f32
// B x [T, 2048]).  DiT::load (src/dit.h:104-140), then n_runs calls of
// DiT::forward (src/dit.h:315-388: the graph of dit_build_graph, :249-287,
// through ggml_backend_sched_graph_compute) on the same inputs, each timed on
// the host clock around the whole call (input uploads, the host timestep
// embedding, the graph, the velocity read-back).  Writes:
//   velocity.bin      f32 B x [T, 128] of the first run;
//   velocity_last.bin the same of the last run;
//   head.bin          hidden_after_preprocess [2304, T, B], then
//                     hidden_after_proj_in [2048, T, B], then the blocks'
//                     input (the timestep token prepended) [2048, T + 1, B],
//                     then layer0_sa_output [2048, T + 1, B];
//   blocks.bin        every block's output x [2048, T + 1, B], blocks 0..35;
//   tail.bin          proj_out's output [128, T, B] (the MUL_MAT of out_w).
// The probes after the last run are graph tensors read in place: the named
// outputs of dit_build_graph (src/dit.h:261-277) and, for the blocks that
// name none, the residual ADD that ends dit_block (:246), found by its
// ff_out projection weight.  The host ggml layer's allocator gives every
// graph tensor its own memory (no reuse), which the driver checks (the
// block outputs must not overlap).  Prints one JSON line with the per-run
// times and the backend's graph statistics.
#include "dit.h"

#include "cpu_standin.h"

#include <chrono>

using namespace refdrv;

static ggml_tensor * named(ggml_cgraph * g, const char * name) {
    ggml_tensor * t = ggml_graph_get_tensor(g, name);
    if (!t) {
        fprintf(stderr, "[driver] graph tensor %s not found\n", name);
        exit(6);
    }
    return t;
}

static void append(std::vector<uint8_t> & out, const ggml_tensor * t) {
    const size_t n = ggml_nbytes(t), o = out.size();
    out.resize(o + n);
    ggml_backend_tensor_get(t, out.data() + o, 0, n);
}

int main(int argc, char ** argv) {
    if (argc != 7) {
        fprintf(stderr, "usage: %s <dit.gguf> <io_dir> <T> <B> <t> <n_runs>\n", argv[0]);
        return 2;
    }
    const std::string dir    = argv[2];
    const int         T      = atoi(argv[3]);
    const int         B      = atoi(argv[4]);
    const float       tt     = (float) atof(argv[5]);
    const int         n_runs = atoi(argv[6]);
    register_cpu_standin();

    static DiT dit;
    if (!dit.load(argv[1])) {
        fprintf(stderr, "[driver] DiT::load failed\n");
        return 3;
    }
    std::vector<float> xt   = read_vec<float>(dir + "/xt.bin");
    std::vector<float> cond = read_vec<float>(dir + "/cond.bin");
    if (xt.size() < (size_t) B * T * DiT::IN_CH || cond.size() < (size_t) B * T * DiT::COND_DIM) {
        fprintf(stderr, "[driver] input files too short\n");
        return 2;
    }

    const size_t       nv = (size_t) B * T * DiT::IN_CH;
    std::vector<float> v0(nv), v(nv);
    std::vector<double> ms;
    bool               same = true;
    for (int r = 0; r < n_runs; r++) {
        const auto t0 = std::chrono::steady_clock::now();
        if (!dit.forward(xt.data(), cond.data(), T, B, tt, r == 0 ? v0.data() : v.data())) {
            fprintf(stderr, "[driver] forward (run %d) failed\n", r);
            return 4;
        }
        const auto t1 = std::chrono::steady_clock::now();
        ms.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count());
        if (r > 0 && memcmp(v.data(), v0.data(), nv * sizeof(float)) != 0) {
            same = false;
        }
    }
    write_bytes(dir + "/velocity.bin", v0.data(), nv * 4);
    write_bytes(dir + "/velocity_last.bin", (n_runs > 1 ? v : v0).data(), nv * 4);

    ggml_cgraph *        g = dit.graph;
    std::vector<uint8_t> head;
    ggml_tensor *        pre    = named(g, "hidden_after_preprocess");
    ggml_tensor *        pin    = named(g, "hidden_after_proj_in");
    ggml_tensor *        sa0    = named(g, "layer0_sa_output");
    ggml_tensor *        first  = nullptr;  // the concat [temb, proj_in] that block 0 normalises
    ggml_tensor *        y_tail = nullptr;
    ggml_tensor *        outs[DiT::N_LAYERS] = {};
    for (int i = 0; i < ggml_graph_n_nodes(g); i++) {
        ggml_tensor * n = ggml_graph_node(g, i);
        if (!first && n->op == GGML_OP_NORM) {
            first = n->src[0];
        }
        if (n->op == GGML_OP_MUL_MAT && n->src[0] == dit.out_w) {
            y_tail = n;
        }
        // x + (ff_out(act) + ff_out_b): the block's last node
        if (n->op == GGML_OP_ADD && n->src[1] && n->src[1]->op == GGML_OP_ADD && n->src[1]->src[0] &&
            n->src[1]->src[0]->op == GGML_OP_MUL_MAT) {
            for (int l = 0; l < DiT::N_LAYERS; l++) {
                if (n->src[1]->src[0]->src[0] == dit.blocks[l].ff_out_w) {
                    outs[l] = n;
                }
            }
        }
    }
    if (!first || !y_tail || first->op != GGML_OP_CONCAT) {
        fprintf(stderr, "[driver] graph structure not as expected\n");
        return 6;
    }
    for (int l = 0; l < DiT::N_LAYERS; l++) {
        if (!outs[l]) {
            fprintf(stderr, "[driver] no output node for block %d\n", l);
            return 6;
        }
        for (int m = 0; m < l; m++) {
            const char * a = (const char *) outs[l]->data, *b = (const char *) outs[m]->data;
            if (a < b + ggml_nbytes(outs[m]) && b < a + ggml_nbytes(outs[l])) {
                fprintf(stderr, "[driver] block outputs %d and %d share memory\n", m, l);
                return 7;
            }
        }
    }
    append(head, pre);
    append(head, pin);
    append(head, first);
    append(head, sa0);
    write_bytes(dir + "/head.bin", head.data(), head.size());
    {
        std::vector<uint8_t> blocks;
        for (int l = 0; l < DiT::N_LAYERS; l++) {
            append(blocks, outs[l]);
        }
        write_bytes(dir + "/blocks.bin", blocks.data(), blocks.size());
    }
    {
        std::vector<uint8_t> tail;
        append(tail, y_tail);
        write_bytes(dir + "/tail.bin", tail.data(), tail.size());
    }
    // the named probes are the same tensors as the blocks' outputs found above
    const int probe_layers[] = { 0, 6, 12, 18, DiT::N_LAYERS - 1 };
    for (int l : probe_layers) {
        char nm[64];
        snprintf(nm, sizeof(nm), "hidden_after_layer%d", l);
        if (named(g, nm) != outs[l]) {
            fprintf(stderr, "[driver] %s is not block %d's output\n", nm, l);
            return 6;
        }
    }

    int64_t            replays = -1, eager = -1;
    ggml_backend_dev_t dev     = ggml_backend_get_device(dit.backend);
    ggml_backend_reg_t reg     = dev ? ggml_backend_dev_backend_reg(dev) : nullptr;
    if (reg) {
        auto stats = (void (*)(ggml_backend_t, int64_t *, int64_t *)) ggml_backend_reg_get_proc_address(
            reg, "ggml_backend_mi355x_graph_stats");
        if (stats) {
            stats(dit.backend, &replays, &eager);
        }
    }
    printf("{\"backend\": \"%s\", \"nodes\": %d, \"runs_identical\": %s, \"replays\": %lld, \"eager\": %lld, "
           "\"ms\": [",
           ggml_backend_name(dit.backend), ggml_graph_n_nodes(g), same ? "true" : "false", (long long) replays,
           (long long) eager);
    for (size_t i = 0; i < ms.size(); i++) {
        printf("%s%.3f", i ? ", " : "", ms[i]);
    }
    printf("]}\n");
    fflush(stdout);
    dit.free();
    return 0;
}

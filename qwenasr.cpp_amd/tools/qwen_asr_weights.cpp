// Counterpart of the reference's tools/qwen-asr-weights.cpp: opens a GGUF file through the mapped
// reader of gguf-model.h and prints its tensor directory (key=value lines, the reference's keys), and
// runs the same write-then-read fixture self-test (tools/qwen-asr-weights.cpp:58-143) with this
// build's GGUF writer.  --write-synthetic writes a seeded synthetic text model as a checkpoint the
// text-decoder drop-in loads (the synthetic counterpart of convert.py).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include <unistd.h>

#include <algorithm>

#include "gguf-model.h"
#include "qwenasr_amd.h"

namespace {

void usage(const char * argv0) {
    std::cerr << "Usage: " << argv0 << " model.gguf [--limit N] [--tensor NAME]\n"
              << "       " << argv0 << " --self-test\n"
              << "       " << argv0 << " --write-synthetic out.gguf [--size 0.6b|1.7b] [--layers N] [--vocab N] [--seed S]\n";
}

const char * type_name(ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return "f32";
        case GGML_TYPE_F16: return "f16";
        case GGML_TYPE_BF16: return "bf16";
        default: return "other";
    }
}

std::string shape_string(const std::vector<int64_t> & ne) {
    std::ostringstream ss;
    ss << "[";
    for (size_t i = 0; i < ne.size(); ++i) ss << (i ? "," : "") << ne[i];
    ss << "]";
    return ss.str();
}

void print_tensor(const QwenAsrGgufTensorView & t, const std::string & prefix) {
    std::cout << prefix << "name=" << t.name << "\n"
              << prefix << "type=" << type_name(t.type) << "\n"
              << prefix << "shape=" << shape_string(t.ne) << "\n"
              << prefix << "bytes=" << t.nbytes << "\n"
              << prefix << "offset=" << t.offset << "\n";
    if (t.type == GGML_TYPE_F32 && t.nbytes >= sizeof(float) && t.data) {
        float v = 0.0f;
        std::memcpy(&v, t.data, sizeof(float));
        std::cout << prefix << "first_f32=" << v << "\n";
    }
}

bool parse_long(const char * s, long lo, long hi, long * out) {
    char * end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (!end || *end != '\0' || v < lo || v > hi) return false;
    *out = v;
    return true;
}

int self_test() {
    const std::string path = "/tmp/qwenasr-weights-fixture-" + std::to_string(static_cast<long>(getpid())) + ".gguf";
    const float values[4] = {1.25f, -2.5f, 3.75f, 4.5f};
    QwenAsrGgufWriter w;
    qwenasr_gguf_writer_set_str(&w, "general.name", "qwenasr tensor fixture");
    qwenasr_gguf_writer_add_tensor(&w, "fixture.weight", GGML_TYPE_F32, {4}, values);
    std::string error;
    if (!qwenasr_gguf_writer_write(w, path.c_str(), &error)) {
        std::cerr << error << "\n";
        return 1;
    }
    QwenAsrGgufModel model{};
    if (!qwenasr_gguf_model_open(path.c_str(), &model, &error)) {
        std::remove(path.c_str());
        std::cerr << error << "\n";
        return 1;
    }
    QwenAsrGgufTensorView t;
    if (!qwenasr_gguf_model_tensor_by_name(model, "fixture.weight", &t, &error)) {
        qwenasr_gguf_model_close(&model);
        std::remove(path.c_str());
        std::cerr << error << "\n";
        return 1;
    }
    float got[4] = {};
    std::memcpy(got, t.data, sizeof(got));
    std::string name;
    const bool ok = t.type == GGML_TYPE_F32 && t.ne == std::vector<int64_t>({4}) && t.nbytes == sizeof(values) &&
                    std::memcmp(got, values, sizeof(values)) == 0 && model.data_offset % 32 == 0 &&
                    qwenasr_gguf_model_get_str(model, "general.name", &name) && name == "qwenasr tensor fixture";
    std::cout << "file_size=" << model.file_size << "\n"
              << "data_offset=" << model.data_offset << "\n"
              << "tensors=" << qwenasr_gguf_model_tensor_count(model) << "\n";
    print_tensor(t, "tensor.0.");
    qwenasr_gguf_model_close(&model);
    std::remove(path.c_str());
    if (!ok) {
        std::cerr << "tensor fixture data mismatch\n";
        return 1;
    }
    std::cout << "status=self-test-ok\n";
    return 0;
}

}  // namespace

int main(int argc, char ** argv) {
    if (argc < 2) {
        usage(argv[0]);
        return 2;
    }
    long limit = 8, n_layers = -1, vocab = -1, seed = 20260101;
    std::string path, tensor_name, write_path, size = "0.6b";
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&](const char * what) -> const char * {
            if (++i >= argc) {
                std::cerr << a << " requires " << what << "\n";
                std::exit(2);
            }
            return argv[i];
        };
        if (a == "-h" || a == "--help") {
            usage(argv[0]);
            return 0;
        }
        if (a == "--self-test") return self_test();
        if (a == "--limit") {
            if (!parse_long(next("a non-negative integer"), 0, 1000000, &limit)) {
                std::cerr << "--limit requires a non-negative integer\n";
                return 2;
            }
        } else if (a == "--tensor") {
            tensor_name = next("a tensor name");
        } else if (a == "--write-synthetic") {
            write_path = next("a path");
        } else if (a == "--size") {
            size = next("0.6b or 1.7b");
        } else if (a == "--layers") {
            if (!parse_long(next("an integer"), 1, 1000, &n_layers)) {
                std::cerr << "--layers requires a positive integer\n";
                return 2;
            }
        } else if (a == "--vocab") {
            if (!parse_long(next("an integer"), 1, 1 << 24, &vocab)) {
                std::cerr << "--vocab requires a positive integer\n";
                return 2;
            }
        } else if (a == "--seed") {
            if (!parse_long(next("an integer"), 0, 0x7fffffffL, &seed)) {
                std::cerr << "--seed requires a non-negative integer\n";
                return 2;
            }
        } else if (!path.empty()) {
            std::cerr << "only one GGUF path is supported\n";
            return 2;
        } else {
            path = a;
        }
    }

    if (!write_path.empty()) {
        qa_text_config cfg{};
        if (size == "1.7b") cfg = {28, 2048, 16, 8, 128, 6144, 151936, 1000000.0f, 1e-6f};
        else if (size == "0.6b") cfg = {28, 1024, 16, 8, 128, 3072, 151936, 1000000.0f, 1e-6f};
        else {
            std::cerr << "--size requires 0.6b or 1.7b\n";
            return 2;
        }
        if (n_layers > 0) cfg.n_layers = static_cast<int32_t>(n_layers);
        if (vocab > 0) cfg.vocab = static_cast<int32_t>(vocab);
        qa_model * m = nullptr;
        if (qa_model_synthetic(&cfg, static_cast<uint64_t>(seed), &m) != QA_OK ||
            qa_gguf_write_model(m, write_path.c_str()) != QA_OK) {
            std::cerr << qa_last_error() << "\n";
            qa_model_free(m);
            return 1;
        }
        qa_model_free(m);
        std::cout << "wrote=" << write_path << "\n" << "layers=" << cfg.n_layers << "\n" << "hidden=" << cfg.hidden
                  << "\n" << "vocab=" << cfg.vocab << "\n";
        return 0;
    }
    if (path.empty()) {
        std::cerr << "GGUF path is required\n";
        return 2;
    }
    QwenAsrGgufModel model{};
    std::string error;
    if (!qwenasr_gguf_model_open(path.c_str(), &model, &error)) {
        std::cerr << error << "\n";
        return 1;
    }
    std::cout << "file_size=" << model.file_size << "\n"
              << "data_offset=" << model.data_offset << "\n"
              << "tensors=" << qwenasr_gguf_model_tensor_count(model) << "\n";
    if (!tensor_name.empty()) {
        QwenAsrGgufTensorView t;
        if (!qwenasr_gguf_model_tensor_by_name(model, tensor_name.c_str(), &t, &error)) {
            qwenasr_gguf_model_close(&model);
            std::cerr << error << "\n";
            return 1;
        }
        print_tensor(t, "tensor.");
    } else {
        const int64_t n = std::min<int64_t>(qwenasr_gguf_model_tensor_count(model), limit);
        for (int64_t i = 0; i < n; ++i) {
            QwenAsrGgufTensorView t;
            if (!qwenasr_gguf_model_tensor_by_index(model, i, &t, &error)) {
                qwenasr_gguf_model_close(&model);
                std::cerr << error << "\n";
                return 1;
            }
            print_tensor(t, "tensor." + std::to_string(i) + ".");
        }
    }
    qwenasr_gguf_model_close(&model);
    return 0;
}

// Test infrastructure only: a C entry layer over the reference's own runtime
// (runtime/src/loader.cpp + executor.cpp, compiled from the reference sources by
// oracle/Makefile into _ref/libggmlref.so), so tests can load a .gguf with the
// reference loader and run it with the reference executor on the CPU — the same
// calls ggmlc's Python runner makes through its binding
// (runtime/bindings/python_bindings.cpp:106-217, python/ggmlc/runtime/runner.py:97-214).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>
#include <unordered_map>

#include "ggmlc/executor.h"
#include "ggmlc/loader.h"

namespace {

thread_local std::string g_err;

struct RefRuntime {
    ggmlc::SerializedModelGraph graph;
    ggmlc::ModelExecutor* ex = nullptr;
};

template <typename F>
int guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

void put_dim(std::string& o, const ggmlc::DimExpr& d, const std::vector<std::string>& syms) {
    static const char* names[] = {"static", "symbol", "add", "sub", "mul", "floordiv", "ceildiv"};
    const int t = (int)d.type;
    if (d.type == ggmlc::DimType::STATIC) {
        o += std::to_string(d.val);
    } else if (d.type == ggmlc::DimType::SYMBOL) {
        o += (d.val >= 0 && d.val < (int64_t)syms.size()) ? syms[d.val] : std::string("?");
    } else {
        o += "(";
        o += names[t];
        o += " ";
        put_dim(o, *d.left, syms);
        o += " ";
        put_dim(o, *d.right, syms);
        o += ")";
    }
}

}  // namespace

extern "C" {

const char* ref_rt_last_error() { return g_err.c_str(); }

void* ref_rt_load(const char* path) {
    RefRuntime* r = new RefRuntime;
    if (guard([&] {
            r->graph = ggmlc::ModelLoader::load_from_file(path);
            r->ex = new ggmlc::ModelExecutor(r->graph, "cpu");
        })) {
        delete r;
        return nullptr;
    }
    return r;
}

void ref_rt_free(void* h) {
    RefRuntime* r = static_cast<RefRuntime*>(h);
    if (!r) return;
    delete r->ex;
    delete r;
}

// One line per item as the reference loader sees the file:
//   S <symbol>                       symbol table, in order
//   I <tid> / O <tid> / P <tid>      inputs, outputs, parameters
//   T <tid> <name> <type> <storage> <ne0> <ne1> <ne2> <ne3> <data_size>
//   N <id> <opcode> <name> <inputs,> <outputs,> <key=int:double;...>   (attributes sorted)
//   M <key> <value>                  string metadata except the graph spec
// Returns the bytes needed (call again with a larger buffer when it exceeds cap).
int64_t ref_rt_describe(void* h, char* buf, int64_t cap) {
    RefRuntime* r = static_cast<RefRuntime*>(h);
    const auto& g = r->graph;
    std::string o;
    for (const auto& s : g.symbol_table) o += "S " + s + "\n";
    for (auto t : g.inputs) o += "I " + std::to_string(t) + "\n";
    for (auto t : g.outputs) o += "O " + std::to_string(t) + "\n";
    for (auto t : g.parameters) o += "P " + std::to_string(t) + "\n";
    std::vector<uint32_t> ids;
    for (const auto& p : g.tensors) ids.push_back(p.first);
    std::sort(ids.begin(), ids.end());
    for (auto id : ids) {
        const auto& t = g.tensors.at(id);
        o += "T " + std::to_string(id) + " " + t.name + " " + std::to_string((int)t.type) + " " +
             std::to_string((int)t.storage);
        for (int i = 0; i < 4; ++i) {
            o += " ";
            put_dim(o, *t.ne[i], g.symbol_table);
        }
        o += " " + std::to_string(t.data_size) + "\n";
    }
    for (const auto& op : g.ops) {
        o += "N " + std::to_string(op.id) + " " + std::to_string(op.opcode) + " " + (op.name.empty() ? "-" : op.name) + " ";
        for (size_t i = 0; i < op.inputs.size(); ++i) o += (i ? "," : "") + std::to_string(op.inputs[i]);
        o += " ";
        for (size_t i = 0; i < op.outputs.size(); ++i) o += (i ? "," : "") + std::to_string(op.outputs[i]);
        o += " ";
        std::vector<std::string> keys;
        for (const auto& a : op.attributes) keys.push_back(a.first);
        std::sort(keys.begin(), keys.end());
        for (const auto& k : keys) {
            char tmp[64];
            snprintf(tmp, sizeof(tmp), "%.9g", op.float_attributes.at(k));
            o += k + "=" + std::to_string(op.attributes.at(k)) + ":" + tmp + ";";
        }
        o += "\n";
    }
    std::vector<std::string> mkeys;
    for (const auto& m : g.metadata_str)
        if (m.first != "ggmlc.graph_spec") mkeys.push_back(m.first);
    std::sort(mkeys.begin(), mkeys.end());
    for (const auto& k : mkeys) o += "M " + k + " " + g.metadata_str.at(k) + "\n";
    const int64_t need = (int64_t)o.size() + 1;
    if (buf && cap >= need) std::memcpy(buf, o.c_str(), (size_t)need);
    return need;
}

int ref_rt_init_kv(void* h, int64_t max_ctx) {
    return guard([&] { static_cast<RefRuntime*>(h)->ex->init_kv_cache(max_ctx); });
}

int ref_rt_reset_kv(void* h) {
    return guard([&] { static_cast<RefRuntime*>(h)->ex->reset_kv_cache(); });
}

// prepare(symbols) + set_input per (tid, bytes) + run(n_threads)
int ref_rt_run(void* h, const char* const* sym_names, const int64_t* sym_vals, int n_sym, const uint32_t* in_tids,
               const void* const* in_data, const int64_t* in_bytes, int n_in, int n_threads) {
    RefRuntime* r = static_cast<RefRuntime*>(h);
    return guard([&] {
        std::unordered_map<std::string, int64_t> env;
        for (int i = 0; i < n_sym; ++i) env[sym_names[i]] = sym_vals[i];
        r->ex->prepare(env, true);
        for (int i = 0; i < n_in; ++i) r->ex->set_input(in_tids[i], in_data[i], (size_t)in_bytes[i]);
        r->ex->run(n_threads);
    });
}

// output tensor tid: ne (4) and its bytes copied into buf (returns the byte count, -1 on error)
int64_t ref_rt_output(void* h, uint32_t tid, int64_t* ne, void* buf, int64_t cap) {
    RefRuntime* r = static_cast<RefRuntime*>(h);
    int64_t n = -1;
    if (guard([&] {
            const auto shp = r->ex->get_tensor_shape(tid);
            for (int i = 0; i < 4; ++i) ne[i] = shp[i];
            n = (int64_t)r->ex->get_tensor_size_bytes(tid);
            if (buf && cap >= n) std::memcpy(buf, r->ex->get_output_data(tid), (size_t)n);
        }))
        return -1;
    return n;
}

}  // extern "C"

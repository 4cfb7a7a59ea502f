// ============================================================================
//  engine.cpp — mars_engine: the JSON-line engine server over the C ABI
//  (protocol of the reference's src/engine_server.cu:9-14, 242-354).
//
//  One JSON object per stdin line, one per stdout line:
//    ADD      {"cmd":"ADD","id":i,"modality":m,"embedding":[...],"timestamp":t} -> {"ok":true}
//    QUERY    {"cmd":"QUERY","embedding":[...],"top_k":10,"bfs_max_hops":2,
//              "modality_filter":-1,"timestamp":t}
//             -> {"results":[{"id","score","modality","hops"}...],"gpu_ms":x}
//    DELETE   {"cmd":"DELETE","id":i}                        -> {"ok":true}
//    STATS    {"cmd":"STATS"}                                -> {"n","edges","vram_mb"}
//    SAVE     {"cmd":"SAVE","path":"..."}                    -> {"ok":true} (MARS v1 file)
//    LOAD     {"cmd":"LOAD","path":"..."}                    -> {"ok":true,"n":N}
//    SHUTDOWN {"cmd":"SHUTDOWN"}                             -> {"ok":true}, then exit
//  Errors: {"ok":false,"error":"..."}.
//
//  The graph lives on the device: ADD appends through the streaming insert, an ADD
//  of an existing id rewrites its row in place, and an id past the end first appends
//  zero rows for the gap, as the reference's host graph grows; embeddings are
//  L2-normalised on arrival (fp32 sum of squares in order, sqrt + 1e-8, as the
//  reference). DELETE leaves a tombstone (zero row, timestamp -1).
//  Edges (--edges):
//    nsn  (default) the reference server's: before a QUERY, the NSN graph
//         (build_nsn_edges(6, 0.15), memory_graph.cpp:102-189) is rebuilt over all
//         nodes on the first query, once the node count has doubled, or once more
//         than 1000 nodes arrived since the last build (engine_server.cu:187-200);
//         only the CSR is replaced, the rows stay resident. Nodes added since the last
//         build have no edges yet.
//    knn  each ADD links the new node to its --knn nearest neighbours by cosine.
//  QUERY runs the certified path (fp16 scan, answers bit-identical to the fp32 path;
//  a query it cannot certify is answered by the fp32 path) with the reference server's
//  decay 1e-8 and hop decay 0.5. SAVE / LOAD write and read MARS v1 checkpoints (the
//  reference's are stubs). No GPU call is made before the first ADD or LOAD.
//
//  Usage: mars_engine [--dim 768] [--capacity 1000000] [--edges nsn|knn] [--knn 8]
// ============================================================================
#include "mars_amd.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <map>
#include <string>
#include <vector>

namespace {

// ---- a flat JSON object: string, number, bool and number-array values ------------
struct Json {
    std::map<std::string, std::string> str;
    std::map<std::string, double> num;
    std::map<std::string, std::vector<float>> arr;

    double number(const char* k, double dflt) const {
        const auto it = num.find(k);
        return it == num.end() ? dflt : it->second;
    }
    std::string string(const char* k) const {
        const auto it = str.find(k);
        return it == str.end() ? std::string() : it->second;
    }
};

class Parser {
public:
    explicit Parser(const std::string& s) : s_(s) {}

    bool object(Json* out) {
        ws();
        if (!eat('{')) return false;
        ws();
        if (eat('}')) return tail();
        for (;;) {
            std::string key;
            ws();
            if (!quoted(&key)) return false;
            ws();
            if (!eat(':')) return false;
            ws();
            if (!value(key, out)) return false;
            ws();
            if (eat('}')) return tail();
            if (!eat(',')) return false;
        }
    }

private:
    bool tail() {
        ws();
        return i_ == s_.size();
    }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\r' || s_[i_] == '\n')) ++i_;
    }
    bool eat(char c) {
        if (i_ < s_.size() && s_[i_] == c) {
            ++i_;
            return true;
        }
        return false;
    }
    bool quoted(std::string* out) {
        if (!eat('"')) return false;
        out->clear();
        while (i_ < s_.size() && s_[i_] != '"') {
            char c = s_[i_++];
            if (c == '\\' && i_ < s_.size()) {
                const char e = s_[i_++];
                c = e == 'n' ? '\n' : e == 't' ? '\t' : e;     // \" \\ \/ and the common escapes
            }
            out->push_back(c);
        }
        return eat('"');
    }
    bool number(double* v) {
        const char* p = s_.c_str() + i_;
        char* end = nullptr;
        *v = std::strtod(p, &end);
        if (end == p) return false;
        i_ += size_t(end - p);
        return true;
    }
    // array elements: decimal -> float in one rounding, as the reference's strtof
    bool number_f(float* v) {
        const char* p = s_.c_str() + i_;
        char* end = nullptr;
        *v = std::strtof(p, &end);
        if (end == p) return false;
        i_ += size_t(end - p);
        return true;
    }
    bool word(const char* w) {
        const size_t n = std::strlen(w);
        if (s_.compare(i_, n, w) != 0) return false;
        i_ += n;
        return true;
    }
    bool value(const std::string& key, Json* out) {
        if (i_ >= s_.size()) return false;
        const char c = s_[i_];
        if (c == '"') return quoted(&out->str[key]);
        if (c == '[') {
            ++i_;
            std::vector<float>& a = out->arr[key];
            ws();
            if (eat(']')) return true;
            for (;;) {
                float v;
                ws();
                if (!number_f(&v)) return false;
                a.push_back(v);
                ws();
                if (eat(']')) return true;
                if (!eat(',')) return false;
            }
        }
        if (word("true")) { out->num[key] = 1.0; return true; }
        if (word("false")) { out->num[key] = 0.0; return true; }
        if (word("null")) return true;
        double v;
        if (!number(&v)) return false;
        out->num[key] = v;
        return true;
    }

    const std::string& s_;
    size_t i_ = 0;
};

std::string escape(const std::string& s) {
    std::string o;
    for (const char c : s) {
        if (c == '"' || c == '\\') o.push_back('\\');
        o.push_back(c == '\n' ? ' ' : c);
    }
    return o;
}

void respond(const std::string& line) {
    std::fputs(line.c_str(), stdout);
    std::fputc('\n', stdout);
    std::fflush(stdout);
}

void respond_error(const std::string& msg) { respond("{\"ok\":false,\"error\":\"" + escape(msg) + "\"}"); }

std::string last_error() {
    const char* m = mars_last_error();
    return m ? m : "error";
}

// ---- server state ------------------------------------------------------------------
struct Engine {
    int32_t dim = 768;
    int32_t capacity = 1000000;
    int32_t knn = 8;
    bool nsn = true;                 // --edges nsn: the reference server's rebuild policy
    mars_graph* g = nullptr;
    mars_ctx* ctx = nullptr;
    int32_t n = 0;
    std::vector<int32_t> mods;       // host copy of every node's modality (the NSN bridges read it)
    int32_t last_rebuild = 0;        // node count of the last NSN build (0: none yet)

    ~Engine() { drop(); }

    void drop() {
        if (ctx) mars_ctx_destroy(ctx);
        if (g) mars_graph_destroy(g);
        ctx = nullptr;
        g = nullptr;
        n = 0;
    }

    // Device graph from host arrays (the first ADD, or LOAD), with room for capacity nodes.
    int create(int32_t nodes, int32_t edges, const int32_t* ro, const int32_t* col, const float* emb,
               const int32_t* mods, const float* ts) {
        drop();
        mars_graph_desc d{};
        d.num_nodes = nodes;
        d.num_edges = edges;
        d.embedding_dim = dim;
        d.row_offsets = ro;
        d.col_indices = col;
        d.embeddings = emb;
        d.modalities = mods;
        d.timestamps = ts;
        d.capacity_nodes = capacity > nodes ? capacity : nodes;
        int rc = mars_graph_create(&d, &g);
        if (rc == MARS_OK) rc = mars_graph_enable_fp16(g);
        if (rc == MARS_OK) rc = mars_ctx_create(d.capacity_nodes, dim, 64, MARS_CTX_TIMING | MARS_CTX_CERTIFIED, &ctx);
        if (rc != MARS_OK) {
            drop();
            return rc;
        }
        n = nodes;
        this->mods.assign(mods, mods + nodes);
        last_rebuild = edges > 0 ? nodes : 0;        // a loaded graph keeps its edges until the next rebuild
        return MARS_OK;
    }

    // ensure_device of the reference server (engine_server.cu:187-200): the NSN graph over
    // all nodes on the first query, after the node count doubled, or after 1000 more.
    int ensure_edges() {
        if (!nsn || !g || n <= 0) return MARS_OK;
        if (last_rebuild != 0 && n < 2 * last_rebuild && n - last_rebuild <= 1000) return MARS_OK;
        int64_t bound = 0;
        int rc = mars_nsn_edges(n, mods.data(), 6, 0.15, MARS_NSN_ALL, nullptr, nullptr, 0, &bound);
        if (rc != MARS_OK) return rc;
        std::vector<int32_t> ro(size_t(n) + 1), col(size_t(bound > 0 ? bound : 1));
        int64_t ne = 0;
        rc = mars_nsn_edges(n, mods.data(), 6, 0.15, MARS_NSN_ALL, ro.data(), col.data(), int64_t(col.size()), &ne);
        if (rc == MARS_OK) rc = mars_graph_set_csr(g, int32_t(ne), ro.data(), ne > 0 ? col.data() : nullptr);
        if (rc == MARS_OK) last_rebuild = n;
        return rc;
    }

    // ADD: rows id (normalised) after zero rows for any gap; an existing id is rewritten.
    int add(int32_t id, int32_t modality, const std::vector<float>& e, float t) {
        // L2 normalisation in fp32, accumulated in order, as the reference server's add_node
        std::vector<float> row(e);
        float sq = 0.0f;
        for (const float x : e) sq += x * x;
        const float norm = std::sqrt(sq) + 1e-8f;
        for (float& x : row) x /= norm;
        if (g && id < n) {
            const int rc = mars_graph_set_rows(g, id, 1, row.data(), &modality, &t);
            if (rc == MARS_OK) this->mods[size_t(id)] = modality;
            return rc;
        }
        const int32_t first = g ? n : 0;
        const int32_t count = id - first + 1;
        std::vector<float> rows(size_t(count) * size_t(dim), 0.0f);
        std::vector<int32_t> mods(size_t(count), MARS_MOD_TEXT);
        std::vector<float> ts(size_t(count), 0.0f);
        std::copy(row.begin(), row.end(), rows.end() - dim);
        mods.back() = modality;
        ts.back() = t;
        if (!g) {
            std::vector<int32_t> ro(size_t(count) + 1, 0);
            return create(count, 0, ro.data(), nullptr, rows.data(), mods.data(), ts.data());
        }
        const int rc = mars_graph_insert(g, count, rows.data(), mods.data(), ts.data(), nullptr,
                                         (!nsn && n >= knn) ? knn : 0, nullptr, nullptr);
        if (rc == MARS_OK) {
            n += count;
            this->mods.insert(this->mods.end(), mods.begin(), mods.end());
        }
        return rc;
    }

    int stats(int32_t* edges) const {
        mars_graph_view v{};
        const int rc = mars_graph_get_view(g, &v);
        *edges = v.num_edges;
        return rc;
    }
};

}  // namespace

int main(int argc, char** argv) {
    Engine eng;
    for (int i = 1; i + 1 < argc; i += 2) {
        if (!std::strcmp(argv[i], "--dim")) eng.dim = std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--capacity")) eng.capacity = std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--knn")) eng.knn = std::atoi(argv[i + 1]);
        else if (!std::strcmp(argv[i], "--edges")) {
            if (!std::strcmp(argv[i + 1], "nsn")) eng.nsn = true;
            else if (!std::strcmp(argv[i + 1], "knn")) eng.nsn = false;
            else eng.knn = -1;                         // rejected below
        }
    }
    if (eng.dim <= 0 || eng.capacity <= 0 || eng.knn < 0 || eng.knn > 16) {
        std::fprintf(stderr, "mars_engine: bad arguments\n");
        return 2;
    }
    // requests are read through iostreams only and responses written through stdio only,
    // so the two need no synchronisation (with it, a 17 KB request is read a character
    // at a time)
    std::ios::sync_with_stdio(false);
    std::cin.tie(nullptr);
    std::fprintf(stderr, "mars_engine: ready (dim=%d, capacity=%d)\n", eng.dim, eng.capacity);
    std::string line;
    while (std::getline(std::cin, line)) {
        while (!line.empty() && (line.back() == '\r' || line.back() == '\n')) line.pop_back();
        if (line.empty()) continue;
        Json j;
        if (!Parser(line).object(&j)) {
            respond_error("malformed JSON");
            continue;
        }
        const std::string cmd = j.string("cmd");
        if (cmd == "ADD") {
            const auto it = j.arr.find("embedding");
            const double id = j.number("id", -1.0);
            if (it == j.arr.end() || int32_t(it->second.size()) != eng.dim) {
                respond_error("embedding dimension mismatch");
            } else if (id < 0.0 || id >= double(eng.capacity)) {
                respond_error("id outside [0, capacity)");
            } else if (eng.add(int32_t(id), int32_t(j.number("modality", 0.0)), it->second,
                               float(j.number("timestamp", 0.0))) != MARS_OK) {
                respond_error(last_error());
            } else {
                respond("{\"ok\":true}");
            }
        } else if (cmd == "QUERY") {
            const auto it = j.arr.find("embedding");
            if (it == j.arr.end() || int32_t(it->second.size()) != eng.dim) {
                respond_error("query embedding dimension mismatch");
                continue;
            }
            if (!eng.g) {
                respond("{\"results\":[]}");
                continue;
            }
            if (eng.ensure_edges() != MARS_OK) {
                respond_error(last_error());
                continue;
            }
            mars_retrieval_config cfg;
            mars_config_default(&cfg);
            cfg.top_k = int32_t(j.number("top_k", 10.0));
            cfg.bfs_max_hops = int32_t(j.number("bfs_max_hops", 2.0));
            cfg.modality_filter = int32_t(j.number("modality_filter", -1.0));
            cfg.time_decay_lambda = 1e-8f;
            cfg.bfs_score_decay = 0.5f;
            const int32_t cap = cfg.top_k > 0 ? cfg.top_k : 1;
            std::vector<mars_query_result> res(size_t(cap < 64 ? 64 : cap));
            int32_t count = 0;
            mars_stats st{};
            const int rc = mars_query(eng.g, eng.ctx, it->second.data(), float(j.number("timestamp", 0.0)), &cfg,
                                      res.data(), int32_t(res.size()), &count, &st);
            if (rc != MARS_OK) {
                respond_error(last_error());
                continue;
            }
            std::string out = "{\"results\":[";
            char buf[160];
            for (int32_t i = 0; i < count && i < int32_t(res.size()); ++i) {
                std::snprintf(buf, sizeof(buf), "%s{\"id\":%d,\"score\":%.6f,\"modality\":%d,\"hops\":%d}",
                              i ? "," : "", res[size_t(i)].node_id, double(res[size_t(i)].score),
                              res[size_t(i)].modality, res[size_t(i)].hops_from_seed);
                out += buf;
            }
            std::snprintf(buf, sizeof(buf), "],\"gpu_ms\":%.3f}", double(st.gpu_ms_total));
            respond(out + buf);
        } else if (cmd == "DELETE") {
            const double id = j.number("id", -1.0);
            if (!eng.g || id < 0.0 || id >= double(eng.n)) {
                respond("{\"ok\":true}");          // as the reference: an unknown id is ignored
                continue;
            }
            std::vector<float> zero(size_t(eng.dim), 0.0f);
            int32_t mod = MARS_MOD_TEXT;
            mars_graph_view v{};
            float ts = -1.0f;
            if (mars_graph_get_view(eng.g, &v) == MARS_OK && v.d_modalities) {
                // the tombstone keeps the node's modality, as the reference's host graph does
                int32_t m = 0;
                if (mars_copy_to_host(&m, static_cast<const int32_t*>(v.d_modalities) + int32_t(id),
                                      sizeof(int32_t)) == MARS_OK)
                    mod = m;
            }
            if (mars_graph_set_rows(eng.g, int32_t(id), 1, zero.data(), &mod, &ts) != MARS_OK)
                respond_error(last_error());
            else
                respond("{\"ok\":true}");
        } else if (cmd == "STATS") {
            int32_t edges = 0;
            double vram_mb = 0.0;
            if (eng.g) {
                if (eng.stats(&edges) != MARS_OK) {
                    respond_error(last_error());
                    continue;
                }
                size_t free_b = 0, total_b = 0;
                if (mars_device_memory(&free_b, &total_b) == MARS_OK) vram_mb = double(total_b - free_b) / 1048576.0;
            }
            char buf[160];
            std::snprintf(buf, sizeof(buf), "{\"n\":%d,\"edges\":%d,\"vram_mb\":%.1f}", eng.n, edges / 2, vram_mb);
            respond(buf);
        } else if (cmd == "SAVE") {
            const std::string path = j.string("path");
            if (path.empty()) respond_error("SAVE needs a path");
            else if (!eng.g) respond_error("no graph to save");
            else if (mars_graph_save(eng.g, path.c_str()) != MARS_OK) respond_error(last_error());
            else respond("{\"ok\":true}");
        } else if (cmd == "LOAD") {
            const std::string path = j.string("path");
            int32_t nn = 0, ne = 0, nd = 0;
            if (path.empty()) {
                respond_error("LOAD needs a path");
                continue;
            }
            if (mars_graph_file_info(path.c_str(), &nn, &ne, &nd) != MARS_OK) {
                respond_error(last_error());
                continue;
            }
            if (nd != eng.dim || nn <= 0 || nn > eng.capacity) {
                respond_error("file holds " + std::to_string(nn) + " nodes of dim " + std::to_string(nd));
                continue;
            }
            std::vector<int32_t> ro(static_cast<size_t>(nn) + 1), col(static_cast<size_t>(ne > 0 ? ne : 1));
            std::vector<int32_t> mods(static_cast<size_t>(nn));
            std::vector<float> emb(static_cast<size_t>(nn) * static_cast<size_t>(nd)), ts(static_cast<size_t>(nn));
            if (mars_graph_file_load(path.c_str(), nn, ne, nd, ro.data(), col.data(), emb.data(), mods.data(),
                                     ts.data()) != MARS_OK ||
                eng.create(nn, ne, ro.data(), col.data(), emb.data(), mods.data(), ts.data()) != MARS_OK) {
                respond_error(last_error());
                continue;
            }
            respond("{\"ok\":true,\"n\":" + std::to_string(nn) + "}");
        } else if (cmd == "SHUTDOWN") {
            respond("{\"ok\":true}");
            break;
        } else {
            respond_error("unknown command");
        }
    }
    std::fprintf(stderr, "mars_engine: shutdown\n");
    return 0;
}

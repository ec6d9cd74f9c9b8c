// CPU driver of the library's host-side layout code (llmplayer_amd/csrc/host_layout.h), built by
// tests/test_host_sanitize.py with g++ under AddressSanitizer and UndefinedBehaviorSanitizer.
// It reads one command per line on stdin and answers one line per command on stdout:
//   repack TYPE ROWS COLS IN OUT      -> "planes off0 off1 off2 off3 pitch0 pitch1 pitch2 pitch3"
//                                        (the packed bytes are written to OUT)
//   relayout H N ROW IN HEADS BACK    -> "ok" (rows_to_heads(IN) to HEADS, heads_to_rows back to BACK)
//   plan POS WINDOW SPLITS            -> "start n rows_per_split splits"
//   splits N HKV NCU PERCU Q8         -> "splits wide"
//   cgroups D SPLITS THREADS BATCH    -> "column groups of the split combine"
//   kgroup D G                        -> "kernel group" (kernel_group)
//   range H N ROW K V QS              -> "ek0 .. ek(H-1) ev0 .. ev(H-1) eq0 .. eq(H-1)": range
//                                        exponents of fp32 rows K, V ([N][H*ROW] floats) and of
//                                        the Q8_0 rows QS (N*H*ROW int8 quants, then the scales)
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <iterator>
#include <sstream>
#include <string>
#include <vector>

#include "host_layout.h"

static std::vector<uint8_t> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<uint8_t>(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

static void write_file(const std::string& path, const void* p, size_t n) {
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(p), (std::streamsize)n);
}

int main() {
    std::string line;
    while (std::getline(std::cin, line)) {
        std::istringstream in(line);
        std::string cmd;
        in >> cmd;
        if (cmd == "repack") {
            int type, rows, cols;
            std::string src, dst;
            in >> type >> rows >> cols >> src >> dst;
            // exactly the GGUF bytes, on the heap, so that any read past them is caught
            std::vector<uint8_t> data = read_file(src);
            std::vector<uint8_t> packed;
            size_t off[4] = {0, 0, 0, 0}, pitch[4] = {0, 0, 0, 0};
            const int n = llmp::repack_weight(type, rows, cols, data.data(), packed, off, pitch);
            write_file(dst, packed.data(), packed.size());
            std::printf("%d %zu %zu %zu %zu %zu %zu %zu %zu\n", n, off[0], off[1], off[2], off[3],
                        pitch[0], pitch[1], pitch[2], pitch[3]);
        } else if (cmd == "relayout") {
            size_t H, n, row;
            std::string src, heads, back;
            in >> H >> n >> row >> src >> heads >> back;
            std::vector<uint8_t> host = read_file(src);
            std::vector<uint8_t> stage(H * n * row), again(H * n * row);
            llmp::rows_to_heads(host.data(), stage.data(), H, n, row);
            llmp::heads_to_rows(stage.data(), again.data(), H, n, row);
            write_file(heads, stage.data(), stage.size());
            write_file(back, again.data(), again.size());
            std::printf("ok\n");
        } else if (cmd == "plan") {
            int pos, window, splits;
            in >> pos >> window >> splits;
            const llmp::StepPlan p = llmp::plan_step(pos, window, splits);
            std::printf("%d %d %d %d\n", p.start, p.n, p.rows_per_split, p.splits);
        } else if (cmd == "cgroups") {
            int d, splits, threads, batch;
            in >> d >> splits >> threads >> batch;
            std::printf("%d\n", llmp::reduce_column_groups(d, splits, threads, batch));
        } else if (cmd == "splits") {
            int n, hkv, ncu, per_cu, q8;
            in >> n >> hkv >> ncu >> per_cu >> q8;
            bool wide = false;
            const int s = llmp::default_splits(n, hkv, ncu, per_cu, q8 != 0, &wide);
            std::printf("%d %d\n", s, wide ? 1 : 0);
        } else if (cmd == "kgroup") {
            int d, g;
            in >> d >> g;
            std::printf("%d\n", llmp::kernel_group(d, g));
        } else if (cmd == "range") {
            size_t H, n, row;
            std::string ks, vs, qs;
            in >> H >> n >> row >> ks >> vs >> qs;
            std::vector<uint8_t> kb = read_file(ks), vb = read_file(vs), qb = read_file(qs);
            std::vector<float> k(kb.size() / 4), v(vb.size() / 4);
            std::memcpy(k.data(), kb.data(), kb.size());
            std::memcpy(v.data(), vb.data(), vb.size());
            const size_t nq = n * H * row;
            std::vector<int8_t> q(nq);
            std::vector<float> sc(nq / 32);
            std::memcpy(q.data(), qb.data(), nq);
            std::memcpy(sc.data(), qb.data() + nq, sc.size() * 4);
            std::vector<int> ek(H, 0), ev(H, 0), eq(H, 0);
            llmp::range_exp_rows(k.data(), v.data(), H, n, row, ek.data(), ev.data());
            llmp::range_exp_rows_q8(q.data(), sc.data(), H, n, row, eq.data());
            for (size_t h = 0; h < H; ++h) std::printf("%d ", ek[h]);
            for (size_t h = 0; h < H; ++h) std::printf("%d ", ev[h]);
            for (size_t h = 0; h < H; ++h) std::printf("%d%s", eq[h], h + 1 < H ? " " : "\n");
        } else if (!cmd.empty()) {
            std::printf("unknown command %s\n", cmd.c_str());
            return 2;
        }
        std::fflush(stdout);
    }
    return 0;
}

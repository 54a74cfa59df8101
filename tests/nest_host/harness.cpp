// Runs a generated loop-nest kernel on the CPU: every workgroup and every
// thread of the launch grid in turn (in launch order, or reversed: a kernel
// whose threads are independent gives the same result either way), over
// buffers read from a file, writing the status word and the buffers back. Built with -include hip_host_shim.h
// and -DMLK_NEST_SRC="<generated source>". Test infrastructure only.
#include <stdio.h>
#include <stdlib.h>
#include <vector>

#include MLK_NEST_SRC

mlk_dim3 blockIdx, threadIdx, gridDim, blockDim;

static void readAll(FILE* f, void* p, size_t n) {
    if (n != 0 && fread(p, 1, n, f) != n) {
        fprintf(stderr, "harness: short read\n");
        exit(2);
    }
}

int main(int argc, char** argv) {
    if (argc != 3 && argc != 4) return 2;
    const bool reverse = argc == 4 && argv[3][0] == 'r';
    FILE* f = fopen(argv[1], "rb");
    if (f == nullptr) return 2;
    int32_t nslots = 0;
    readAll(f, &nslots, sizeof(nslots));
    if (nslots < 0 || nslots > 16) return 2;
    std::vector<std::vector<unsigned char>> bufs(static_cast<size_t>(nslots));
    mlk_nest_args a;
    memset(&a, 0, sizeof(a));
    for (int s = 0; s < nslots; ++s) {
        int32_t dt = 0;
        int64_t count = 0;
        readAll(f, &dt, sizeof(dt));
        readAll(f, &count, sizeof(count));
        const size_t bytes = static_cast<size_t>(count) * (dt == 0 ? 4 : (dt == 1 ? 2 : 8));
        bufs[static_cast<size_t>(s)].resize(bytes);
        readAll(f, bufs[static_cast<size_t>(s)].data(), bytes);
        // Exact-size heap blocks: AddressSanitizer flags any access past them.
        a.p[s] = bytes != 0 ? bufs[static_cast<size_t>(s)].data() : nullptr;
        a.n[s] = count;
    }
    mlk_scalars sc;
    readAll(f, sc.v, sizeof(sc.v));
    int64_t elements = 0, total = 0, grid = 0;
    readAll(f, &elements, sizeof(elements));
    readAll(f, &total, sizeof(total));
    readAll(f, &grid, sizeof(grid));
    fclose(f);
    int status = 0;
    a.status = &status;
    a.elements = elements;
    gridDim.x = static_cast<unsigned>(grid);
    const int64_t wg = MLK_NEST_WG;   // the instance's workgroup size (256 unless its launch form sets another)
    blockDim.x = static_cast<unsigned>(wg);
    for (int64_t i = 0; i < grid * wg; ++i) {
        const int64_t g = reverse ? grid * wg - 1 - i : i;
        blockIdx.x = static_cast<unsigned>(g / wg);
        threadIdx.x = static_cast<unsigned>(g % wg);
        mlk_nest(a, sc, total);
    }
    FILE* o = fopen(argv[2], "wb");
    if (o == nullptr) return 2;
    fwrite(&status, sizeof(status), 1, o);
    for (int s = 0; s < nslots; ++s) fwrite(bufs[static_cast<size_t>(s)].data(), 1, bufs[static_cast<size_t>(s)].size(), o);
    fclose(o);
    return 0;
}

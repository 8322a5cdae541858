"""Schedule choices that the measurements fixed, pinned on the generated source (CPU).

- four wavefronts of 2 x 2 MFMA tiles for C4's tall N = 256 products with K >= 512 (a 64 x 64
  output tile per workgroup), while C2's batch-256 products keep four wavefronts of one tile;
- `ANVIL_GEMM_FORCE=<schedule>@MxNxK` changes the products of that shape only;
- row blocks of more than 2048 rows run with 128 lanes per row, shorter ones with 256.
"""
import os
import re

from fixtures import load_ir

from anvil import ir
from anvil.backend import hip


def _source(name):
    prog, data = load_ir(name)
    return hip.generate(prog, seed=data.get("seed", 0))


def _schedules(src):
    """shape -> set of schedule strings of its products ('ksplit 64x64', 'tile 64x64', ...)."""
    out: dict = {}
    for shape, sched in re.findall(r"^// gemm: .*· (\d+x\d+x\d+) · (ksplit \d+x\d+|tile \d+x\d+)", src, re.M):
        out.setdefault(shape, set()).add(sched)
    return out


def test_tall_products_take_two_by_two_tiles():
    s = _schedules(_source("c4_t256_2"))
    assert s["4096x256x1024"] == {"ksplit 64x64"} and s["4096x256x768"] == {"ksplit 64x64"}
    # K = 256: four wavefronts of one tile, K split four ways
    assert s["4096x256x256"] == {"ksplit 32x32"}


def test_batch_256_products_keep_one_tile_per_wavefront():
    s = _schedules(_source("c2_wide_mlp"))
    assert s["256x1024x1024"] == {"ksplit 32x32"}


def test_force_by_shape_touches_that_shape_only(monkeypatch):
    base = _schedules(_source("c4_t256_2"))
    monkeypatch.setenv("ANVIL_GEMM_FORCE", "tile64@4096x256x256")
    forced = _schedules(_source("c4_t256_2"))
    assert forced["4096x256x256"] == {"tile 64x64"}
    assert {k: v for k, v in forced.items() if k != "4096x256x256"} == \
           {k: v for k, v in base.items() if k != "4096x256x256"}


def _rowblock_lanes(src):
    return {(int(rows), int(lanes)) for rows, lanes in re.findall(
        r"rowblock: .*· one workgroup per row, (\d+) rows\n__global__ void __launch_bounds__\((\d+)\)", src)}


def test_rowblock_lanes_follow_the_row_count():
    assert _rowblock_lanes(_source("c4_t256_2")) == {(4096, 128)}
    assert _rowblock_lanes(_source("c2_wide_mlp")) == {(256, 256)}
    assert {lanes for _, lanes in _rowblock_lanes(_source("c4_full2"))} == {256}      # 1024 rows


def _rowblock_plan(prog, data):
    g = hip.HipGen(prog, seed=data.get("seed", 0))
    g.generate()
    (p,) = [p for p in g.plans if p.kind == "rowblock"]
    return p


def test_rowblock_keeps_no_lds_shadow_of_a_buffer_read_before_the_chain_writes_it():
    """rowblock_prior: y = 2x (before the chain), then the chain s = Σ y, y -= s / 256, t = Σ y[..4].
    The `+=` stage reads y's values from the kernel ahead of the launch, so y must stay in memory
    only: an LDS copy of the row would start empty. Also with y taken as a temporary that only the
    chain reads (which alone would make its row slice live in LDS, and its memory store dropped)."""
    prog, data = load_ir("rowblock_prior")
    p = _rowblock_plan(prog, data)
    y = [b for b in prog.buffers if b.name == "y" and b.kind == "var"][0]
    assert y.id in p.before_ids and y.id not in p.shadow
    prog, data = load_ir("rowblock_prior")
    y = [b for b in prog.buffers if b.name == "y" and b.kind == "var"][0]
    y.kind = "temp"
    p = _rowblock_plan(prog, data)
    assert len(p.kernels) == 3 and y.id not in p.shadow and y.id not in p.dead
    assert f"sh{y.id}" not in p.source()


def test_row_chain_stops_before_a_real_product():
    """C4's loss head, log-softmax -> the cross-entropy gradient -> the softmax gradient over 4096
    rows of 96, is one row block that ends where dlogits·W (K = 96, a matrix-core product) begins;
    without the cut the whole chain was refused and ran as four launches (measured on the step
    loop: T = 64 548 -> 541 us, T = 256 1415 -> 1406 us per step)."""
    src = _source("c4_transformer_t256")
    head = [l for l in src.splitlines() if l.startswith("// rowblock: ") and "reduce max j<96" in l]
    assert len(head) == 1 and "x k<256]" not in head[0], head           # the product is not a stage
    assert re.search(r"^// gemm: .*· 4096x256x96 · ", src, re.M)
    import os
    os.environ["ANVIL_HIP_ROWBLOCK_CUT"] = "0"
    try:
        uncut = _source("c4_transformer_t256")
    finally:
        del os.environ["ANVIL_HIP_ROWBLOCK_CUT"]
    assert not any(l.startswith("// rowblock: ") and "reduce max j<96" in l for l in uncut.splitlines())
    assert uncut.count("__global__") == src.count("__global__") + 3


def _split_product_then_nine(dependent):
    """C = Aᵀ·B (64 x 64 outputs, K = 8192: few tiles and a long K, so K is split across workgroups
    and a second launch adds the partial tiles), then eight independent maps; with `dependent`, a
    ninth kernel reads C transposed (not at its own element, so it is no epilogue of the product)."""
    M = N = 64
    K = 8192
    A = ir.Buffer("A", (K, M), "f32", "data")
    B = ir.Buffer("B", (K, N), "f32", "data")
    C = ir.Buffer("C", (M, N), "f32", "var")
    m, n, k = ir.Var("m", M), ir.Var("n", N), ir.Var("k", K)
    g = ir.Kernel([m, n], [ir.Store(C, ir.Affine(0, {m: N, n: 1}), ir.Acc())],
                  red=ir.Reduction([k], "sum", ir.Binary("mul", ir.Load(A, ir.Affine(0, {k: M, m: 1})),
                                                          ir.Load(B, ir.Affine(0, {k: N, n: 1})))), name="g")
    body, bufs = [ir.KernelStmt(g)], [A, B, C]
    for j in range(8):
        L = 1000 + 8 * j                                    # extents apart: no map is another's follower
        x, y = ir.Buffer(f"x{j}", (L,), "f32", "data"), ir.Buffer(f"y{j}", (L,), "f32", "var")
        i = ir.Var("i", L)
        body.append(ir.KernelStmt(ir.Kernel([i], [ir.Store(y, ir.Affine(0, {i: 1}),
                                                            ir.Unary("exp", ir.Load(x, ir.Affine(0, {i: 1}))))],
                                            name=f"e{j}")))
        bufs += [x, y]
    if dependent:
        a, b = ir.Var("a", M), ir.Var("b", N)
        yc = ir.Buffer("yc", (M, N), "f32", "var")
        body.append(ir.KernelStmt(ir.Kernel([a, b], [ir.Store(yc, ir.Affine(0, {a: N, b: 1}),
                                                               ir.Unary("exp", ir.Load(C, ir.Affine(0, {b: N, a: 1}))))],
                                            name="t")))
        bufs.append(yc)
    body += [ir.Print([ir.PrintItem("tensor", buf=x)]) for x in bufs if x.kind == "var"]
    return ir.Program(ir.Block(body), bufs)


def _launch_labels(src):
    return [l.split("// ", 1)[1] for l in src.split("static int anvil_program", 1)[1].splitlines()
            if re.match(r"\s*\{   // ", l) and "on the host" not in l]


def test_a_second_launch_joins_the_next_independent_launch():
    """The partial-tile sum of a K split runs side by side with the next launch when no data passes
    between them: the first launch holds the product and seven maps (eight parts at most), the
    eighth map then shares the sum's launch. When a kernel reads the product, the sum cannot join
    that launch and stays alone (or, with ANVIL_GEMM_FIXUP=1, the product's last workgroup per tile
    adds the partial tiles)."""
    labels = _launch_labels(hip.generate(_split_product_then_nine(False)))
    assert labels[0].startswith("k") and labels[0].count(" map: ") == 7 and " gemm: g" in labels[0]
    assert " map: e7 | " in labels[1] and "gemm-reduce: partial-tile sum + g" in labels[1], labels
    labels = _launch_labels(hip.generate(_split_product_then_nine(True)))
    assert labels[1] == "partial-tile sum + g", labels
    assert "map: e7" in labels[2] and "map: t" in labels[2]
    os.environ["ANVIL_GEMM_FIXUP"] = "1"
    try:
        src = hip.generate(_split_product_then_nine(True))
    finally:
        del os.environ["ANVIL_GEMM_FIXUP"]
    labels = _launch_labels(src)
    assert len(labels) == 2 and "map: e7" in labels[1] and "map: t" in labels[1], labels
    assert "anvil_last_" in src and "gemm-reduce" not in src


def test_c4_and_c5_weight_update_sums_join_the_next_launch(monkeypatch):
    """C5: the loss kernel (one workgroup) runs beside the four weight updates' sums; C4 at T = 256:
    three of the four partial-tile sums run beside the next weight-gradient launch (the last one has
    no launch after it in the step). Measured on the step loops: C5 211.5 -> 209.3 us, C4 1405 ->
    1399 us per step."""
    c5 = _launch_labels(_source("c5_cnn"))
    assert any(l.startswith("k") and "rows: cross_entropy" in l and "gemm-reduce" in l for l in c5), c5
    c4 = _launch_labels(_source("c4_transformer_t256"))
    alone = [l for l in c4 if "partial-tile sum" in l and " gemm: " not in l]
    assert len(alone) == 1, alone
    monkeypatch.setenv("ANVIL_HIP_JOIN", "0")
    assert len(_launch_labels(_source("c5_cnn"))) == len(c5) + 1
    assert len(_launch_labels(_source("c4_transformer_t256"))) == len(c4) + 3


def test_xcd_runs_are_one_contiguous_run_per_xcd(tmp_path):
    """anvil_run_of (hip_rt/anvil_mfma.h), compiled for the host from the header's own text: for
    every grid size up to 3000, the positions of ids 0 .. n - 1 are a permutation of 0 .. n - 1,
    and the ids of each XCD (id mod 8) take one contiguous run of them."""
    import subprocess
    hdr = open(os.path.join(os.path.dirname(hip.__file__), "hip_rt", "anvil_mfma.h")).read()
    start = hdr.index("__device__ __forceinline__ int anvil_run_of")
    fn = hdr[start:hdr.index("\n}\n", start) + 3]
    prog = ("#include <algorithm>\n#include <cstdio>\n#include <vector>\nusing std::min;\n"
            "#define __device__\n#define __forceinline__ inline\n" + fn + r"""
int main() {
    for (int n = 1; n <= 3000; n++) {
        std::vector<int> seen(n, 0), lo(8, n), hi(8, -1), cnt(8, 0);
        for (int L = 0; L < n; L++) {
            const int p = anvil_run_of(L, n);
            if (p < 0 || p >= n || seen[p]++) { printf("n %d L %d p %d\n", n, L, p); return 1; }
            lo[L % 8] = std::min(lo[L % 8], p); hi[L % 8] = std::max(hi[L % 8], p); cnt[L % 8]++;
        }
        for (int x = 0; x < 8; x++)
            if (cnt[x] && hi[x] - lo[x] + 1 != cnt[x]) { printf("n %d xcd %d not contiguous\n", n, x); return 1; }
    }
    return 0;
}
""")
    (tmp_path / "runs.cpp").write_text(prog)
    subprocess.run(["g++", "-O1", "-o", str(tmp_path / "runs"), str(tmp_path / "runs.cpp")], check=True)
    r = subprocess.run([str(tmp_path / "runs")], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout


def test_split_products_walk_xcd_runs(monkeypatch):
    """Every K split across workgroups takes its tile and slice from anvil_run_of (C5: the FC1
    product and both convolutions' weight gradients); ANVIL_GEMM_RUNS=0 keeps launch order, and
    =all adds the two wide grids (the second convolution, the FC1 input gradient)."""
    src = _source("c5_cnn")
    heads = re.findall(r"^// gemm: .*K in \d+ slices.*\n(?:.*\n){1,12}?.*anvil_run_of\(", src, re.M)
    assert src.count("anvil_run_of(") == 1 + 3 and len(heads) == 3
    monkeypatch.setenv("ANVIL_GEMM_RUNS", "0")
    assert _source("c5_cnn").count("anvil_run_of(") == 1
    monkeypatch.setenv("ANVIL_GEMM_RUNS", "all")
    assert _source("c5_cnn").count("anvil_run_of(") == 1 + 3 + 2


def test_weight_gradient_launches_share_partial_tile_lds(monkeypatch):
    """A side-by-side launch of products gives all parts one partial-tile array (a workgroup runs
    one part), sized for the workgroups per CU its longest per-workgroup K measured best with:
    C4 at T = 256 (K = 4096) two, C4 at T = 64 (K = 1024) six, C5 (K = 1320) four; C2's update
    launch (K = 256) keeps each part's own array. Measured on the step loops: 1397 -> 1385 us,
    541 -> 526 us, 201 -> 197 us."""
    def targets(name):
        src = _source(name)
        pools = re.findall(r"^__shared__ float anvil_fl_(\w+)\[(\d+)\];   // the parts' partial tiles, (\d) "
                           r"workgroups per CU", src, re.M)
        for fname, words, _ in pools:              # every part of that launch points at the pool
            body = src[src.index(f"anvil_fl_{fname}["):src.index(f"// fused: ", src.index(f"anvil_fl_{fname}["))]
            assert "__shared__ float anvil_kp_lds" not in body
            assert body.count(f"float *const anvil_kp_lds = anvil_fl_{fname};") >= 2
        return {int(t) for _, _, t in pools}, [int(w) for _, w, _ in pools]
    assert targets("c4_transformer_t256")[0] == {2}
    assert targets("c4_transformer")[0] == {6}
    t5, words = targets("c5_cnn")
    assert t5 == {4} and all(36864 // 2 <= 4 * w <= 36864 for w in words)
    assert targets("c2_wide_mlp")[0] == set()
    # the LDS that lets a CU (160 KB) hold exactly n workgroups
    from anvil.backend import hip_kernels as HK
    for n in range(1, 9):
        b = HK.lds_for(n)
        assert 160 * 1024 // b == n
    monkeypatch.setenv("ANVIL_HIP_FUSED_WGS", "0")
    assert targets("c4_transformer_t256")[0] == set()


def test_layer_norm_folds_into_a_narrow_product(monkeypatch):
    """hip_rowpro: C4's last layer norm runs in the prologue of the 96-wide output product (three
    tile columns: 8.5 us against 6.5 + 5.1 for the product and the norm's own launch), while the
    per-layer norms before y·Wqkv (24 tile columns, each recomputing the rows: 32.5 us against
    23.1 + 5.1) keep their launch; with the column limit raised all five fold."""
    src = _source("c4_transformer_t256")
    labels = _launch_labels(src)
    fold = [l for l in labels if "layer_norm + layer_norm + layer_norm → matmul" in l]
    assert len(fold) == 1 and "matmul+add" in fold[0], fold
    assert src.count("anvil_mm_tile_kpipe_areg<") == 1                  # its one call
    monkeypatch.setenv("ANVIL_HIP_ROWPRO_COLS", "32")
    many = _source("c4_transformer_t256")
    assert many.count("anvil_mm_tile_kpipe_areg<") == 5
    assert len(_launch_labels(many)) == len(labels) - 4
    monkeypatch.setenv("ANVIL_HIP_ROWPRO", "0")
    assert _source("c4_transformer_t256").count("anvil_mm_tile_kpipe_areg<") == 0


def test_cached_rows_move_16_bytes_per_lane(monkeypatch):
    """A row kept in registers (4 elements per lane, side by side and 16-byte aligned) is loaded and
    stored 16 bytes at a time, and a per-column operand the row does not write (layer norm's γ and
    β) likewise: C3's softmax over rows of 4096 54.8 -> 40.5 us (61 -> 83 % of HBM), its layer norm
    11.29 -> 11.09 us. The compiler made separate 4-byte accesses of the element loop."""
    def kernel(name):
        prog, data = load_ir(name)
        src = hip.generate(prog, seed=data.get("seed", 0), library=True)
        i = src.index("// rows: ")
        return src[i:src.index("\n}\n", i)]
    sm = kernel("c3_softmax")
    assert sm.count("*(const anvil_f32x4 *)&") == 1 and sm.count("__builtin_nontemporal_store(w_") == 1
    assert "anvil_store_out(" not in sm
    ln = kernel("c3_layernorm")
    assert ln.count("*(const anvil_f32x4 *)&") == 3          # x, and γ and β in the last stage
    monkeypatch.setenv("ANVIL_HIP_VEC_ROWS", "0")
    assert "anvil_f32x4" not in kernel("c3_softmax")


def test_max_pool_takes_two_outputs_per_lane(monkeypatch):
    """C5's 2 x 2 max-pool (PoolPlan): each lane computes two adjacent outputs, one 16-byte load per
    window row and one 8-byte store per output buffer (C5: 197.6 -> 193.8 us per step); the window's
    elements are combined in the reduction's own order, so the results are the same bits."""
    src = _source("c5_cnn")
    i = src.index("two outputs of the 2-wide window per lane")
    kern = src[i:src.index("\n}\n", i)]
    assert kern.count("*(const anvil_f32x4 *)&") == 2 and kern.count("*(float2 *)&") == 2
    assert "589824 pairs" in kern                       # 128 x 64 x 12 x 12 outputs, in pairs
    monkeypatch.setenv("ANVIL_HIP_POOL", "0")
    assert "two outputs of the 2-wide window" not in _source("c5_cnn")


def test_max_pool_gradient_takes_two_windows_per_lane(monkeypatch):
    """C5's max-pool gradient (then ReLU's) as a map over [n·c·i, u, j, v] with v of extent 2: each
    lane takes two windows' elements along j (four elements), the pre-pool activations in one
    16-byte load, the pooled values and their gradient in one 8-byte load each (shared by the two
    elements of a window), and the result in one 16-byte store; each element's value is the same
    expression as before, so the results are the same bits."""
    src = _source("c5_cnn")
    i = src.index("two 2-wide windows (4 elements) per lane")
    kern = src[i:src.index("\n}\n", i)]
    assert kern.count("*(const anvil_f32x4 *)&") == 1 and kern.count("*(const anvil_f32x2 *)&") == 2
    assert kern.count("*(anvil_f32x4 *)&") == 1 and "w < 1179648u" in kern      # 4718592 elements / 4
    assert "[e >> 1]" in kern and "[e]" in kern
    monkeypatch.setenv("ANVIL_HIP_MAP_PAIRS", "0")
    assert "two 2-wide windows" not in _source("c5_cnn")


def test_four_element_maps_access_16_bytes_at_a_time(monkeypatch):
    """A map with four consecutive elements per lane loads and stores the side-by-side ones as one
    16-byte access each (C4's embedding sum: the positional table row) instead of four 4-byte
    ones that the compiler leaves unmerged."""
    src = _source("c4_transformer_t256")
    heads = [l for l in src.split("\n") if l.startswith("// map:") and "4 elements per lane, 1 loads and 1 stores" in l]
    assert heads
    monkeypatch.setenv("ANVIL_HIP_VEC_MAP", "0")
    assert "stores as one access each" not in _source("c4_transformer_t256")


def test_input_gradient_reads_a_packed_copy_of_the_weights(monkeypatch):
    """C5's input gradient reads W2[o, c, u, v] as A[c, (u, v, o)]; a copy packed in that order
    (32 x 576 floats) is written in the launch before it (beside the max-pool gradient, which does
    not write W2), and the product reads 4 consecutive k with one 16-byte load (ANVIL_LD_KC)."""
    src = _source("c5_cnn")
    assert "// fused: k26278, k26305p side by side" in src
    i = src.index("// conv-dgrad: k26305")
    kern = src[i:src.index("\n}\n", i)]
    assert "the weights from their packed copy (k26305p)" in kern
    assert "anvil_mm_tile_kpipe<4, 1, 2, ANVIL_LD_KC, ANVIL_LD_ANY" in kern
    assert "576LL * (long long)(uint32_t)(t)" in kern
    labels = _launch_labels(src)
    at = next(n for n, l in enumerate(labels) if "k26305p pack" in l)
    assert labels[at + 1] == "∂forward + zero + ∂forward + ∂max" and "∂max_pool2d" in labels[at]
    monkeypatch.setenv("ANVIL_DGRAD_PACK", "0")
    assert "k26305p" not in _source("c5_cnn")


def test_a_pack_runs_alone_after_a_launch_that_writes_its_weights():
    """When the launch before the input gradient writes the weights, the packed copy cannot run
    beside it (it would read them before that launch's writes): it takes a launch of its own."""
    import types
    prog, data = load_ir("c5_cnn")
    g = hip.HipGen(prog, seed=data.get("seed", 0))
    W = prog.buffers[0]
    # the launch before: a map that writes W; the copy reads W
    writer = types.SimpleNamespace(kind="map", grid=lambda: (1, 256), kernels=[ir.Kernel(
        [ir.Var("i", 4)], [ir.Store(W, ir.Affine(0, {}), ir.Const(0.0))], name="w")])
    pack = types.SimpleNamespace(src=W)
    pack.with_threads = lambda t: pack
    g.plans, seg = [writer], [("launch", [], writer)]
    g.launch = lambda p, ind: []
    g.place_pack(pack, seg, "")
    assert pack.own is pack and g.plans == [writer, pack] and seg[-1][2] is pack


def test_a_lone_k_split_adds_its_partial_tiles_in_its_last_workgroup(monkeypatch):
    """With ANVIL_GEMM_FIXUP=1, a K split whose partial-tile sum cannot join the next launch (C5's
    first fully connected product: the row block after it reads its result; C4's 256 x 96 x 4096
    weight gradient, in a launch with three other products) adds the partial tiles in the last
    workgroup of each tile to finish, in slice order, instead of in a second launch; the count of
    finished slices per tile is set back to zero by that workgroup. (Off by default: slower.)"""
    assert "anvil_cnt_" not in _source("c5_cnn")
    monkeypatch.setenv("ANVIL_GEMM_FIXUP", "1")
    src = _source("c5_cnn")
    assert "static __device__ unsigned anvil_cnt_k26677[16];" in src
    assert "atomicAdd(&anvil_cnt_k26677[tile_], 1u) == 17u" in src and "anvil_cnt_k26677[tile_] = 0u;" in src
    assert "k26677r" not in src and "for (int sl = 0; sl < 18; sl++)" in src
    src4 = _source("c4_transformer_t256")
    assert "anvil_cnt_k25543[24]" in src4 and "k25543r" not in src4
    monkeypatch.setenv("ANVIL_GEMM_FIXUP", "0")
    assert "// gemm-reduce: k26677" in _source("c5_cnn")


def test_row_block_stages_of_the_first_wavefront_skip_the_workgroup_barrier(monkeypatch):
    """With ANVIL_ROWBLOCK_WAVESYNC=1, C2's row block (logits, log-softmax, the loss and their
    gradients over 256 rows of 10): the stages that run on at most 64 lanes (one per logit or per
    row) follow each other with a wave-level fence instead of a workgroup barrier; the barrier
    stays before and after them. (Off by default: no faster.)"""
    def barriers(src):
        i = src.index("// rowblock: k1002")
        kern = src[i:src.index("\n}\n", i)]
        return kern.count("__syncthreads();"), kern.count("__builtin_amdgcn_wave_barrier();")
    sync, wave = barriers(_source("c2_full"))
    assert wave == 0
    monkeypatch.setenv("ANVIL_ROWBLOCK_WAVESYNC", "1")
    assert barriers(_source("c2_full")) == (sync - 6, 6)

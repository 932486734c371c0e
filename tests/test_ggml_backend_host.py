"""Host-only checks of the ggml backend core (include/kernelcore/ggml_backend.h): its supports_op
rules (integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp:865-957, weight_shape_ok
:103-109) and the launch sequence graph_compute makes (:706-792) -- which nodes fuse, which are
skipped, which MUL_MATs share a quantized input and run as one concurrent step -- read from
kcGgmlGraphPlan, which walks the nodes exactly as kcGgmlGraphCompute does without a device.

Each fusion rule is checked both ways: the layer graph llama.cpp builds fuses, and a planted
change that ggml_can_fuse or the reference's pattern must reject (a second use of the norm, a
norm that is a graph output or a view, a MUL by a full matrix, rows not a multiple of 256, an
ADD whose result the norm does not read) turns the fusion off."""
import ctypes as C

import pytest

import kernelcore_amd as kc
from kernelcore_amd import ggml_graph as gg


def layer(N=1, n_kv=None, shape=None, **kw):
    g = gg.Graph()
    t = gg.llama_layer(g, shape or gg.LayerShape(**kw), N, n_kv or 40 + N)
    return g, t


def plan(g, **cfg):
    return kc.ggml_graph_plan(g.nodes, **cfg)[0]


ATTN = ["rope_ggml", "rope_ggml", "set_rows_f16", "set_rows_f16", "flash_decode_f16"]  # the reference's launches
# one token: ROPE of q and k and the two SET_ROWS run inside the attention's launch, which also
# quantizes its output (batches: ROPE and SET_ROWS in one launch, then the attention)
ATTN1 = ["rope_flash_decode_q8"]


# ---- graph_compute's walk --------------------------------------------------------------------------------------

@pytest.fixture
def reference_matvecs():
    """The reference's one launch per MUL_MAT node (no fused decode matvec)."""
    kc.set_option("ggml_extra_fusions", 1)
    yield
    kc.set_option("ggml_extra_fusions", 0)


def test_decode_layer_plan():
    g, _ = layer(N=1)
    # one input column: the attention norm inside the q / k / v launch, the FFN norm inside the gate /
    # up / SWIGLU launch, the o and down products each with their residual ADD
    assert plan(g) == (["decode_norm_matvec"] + ATTN1 + ["decode_matvec_add", "decode_norm_swiglu",
                                                         "decode_matvec_add"])


def test_decode_layer_plan_with_one_launch_per_node(reference_matvecs):
    g, _ = layer(N=1)
    assert plan(g) == (["add_norm_q8_f", "[", "matvec_q4k_q8", "matvec_q4k_q8", "matvec_q6k_q8", "]"]
                       + ATTN + ["quantize_q8x4", "matvec_q4k_q8", "add_norm_q8_f",
                                 "[", "matvec_q4k_q8", "matvec_q4k_q8", "]", "silu_mul_q8x4f", "matvec_q6k_q8",
                                 "vector_add"])


def test_matvec_add_fuses_only_when_the_add_is_its_one_use():
    g, t = layer(N=1)
    t["o"].uses = 2  # the o product read again elsewhere: written, then added by the FFN norm
    names = plan(g)
    assert names.count("decode_matvec_add") == 1 and "add_norm_q8_f" in names and "matvec_q4k_q8" in names


@pytest.mark.parametrize("plant", ["output", "second_use"])
def test_norm_inside_the_matvecs_only_when_they_are_its_only_uses(plant):
    g, _ = layer(N=1)
    mul = next(x for x in g.nodes if x.op == kc.GGML_OP["mul"])  # the attention norm's weight
    if plant == "output":
        mul.output = 1
    else:
        mul.uses = 4
    names = plan(g)
    assert names[:2] == ["add_norm_q8_f", "decode_matvec"] and names.count("decode_norm_matvec") == 0


@pytest.mark.parametrize("plant", ["positions", "row_indices", "params"])
def test_rope_and_cache_rows_fuse_only_with_shared_positions_rows_and_parameters(plant):
    g, _ = layer(N=2)
    ropes = [x for x in g.nodes if x.op == kc.GGML_OP["rope"]]
    rows = [x for x in g.nodes if x.op == kc.GGML_OP["set_rows"]]
    if plant == "positions":
        ropes[1].src[1] = C.pointer(g.leaf("i32", [2]))
    elif plant == "row_indices":
        rows[1].src[1] = C.pointer(g.leaf("i64", [2]))
    else:
        ropes[1].op_params[5] = ropes[1].op_params[5] + 1  # another frequency base
    names = plan(g)
    assert "rope_set_rows" not in names and names.count("rope_ggml") == 2 and names.count("set_rows_f16") == 2


@pytest.mark.parametrize("plant", ["q_source", "k_rows", "v_rows", "k_heads"])
def test_rope_enters_the_attention_only_on_the_roped_q_and_cache_views(plant):
    """The ROPE / SET_ROWS nodes run inside one token's attention launch only when the attention reads
    the roped q and views of the two caches from one common row with the caches' row strides and heads
    D halves apart; otherwise ROPE + SET_ROWS stay one launch and the attention another."""
    g, t = layer(N=1)
    fa = next(x for x in g.nodes if x.op == kc.GGML_OP["flash_attn_ext"])
    if plant == "q_source":
        fa.src[0] = C.pointer(g.leaf("f32", [64, 1, 8]))
    elif plant == "k_rows":
        fa.src[1].contents.data = fa.src[1].contents.data + fa.src[1].contents.nb[1]  # a view from row 1
    elif plant == "v_rows":
        fa.src[2].contents.nb[1] = fa.src[2].contents.nb[1] * 2
    else:
        fa.src[1].contents.nb[2] = fa.src[1].contents.nb[2] * 2
    names = plan(g)
    assert "rope_flash_decode_q8" not in names and names[1:3] == ["rope_set_rows", "flash_decode_q8"], names


@pytest.mark.parametrize("plant", ["glu_output", "glu_second_use", "gate_second_use", "up_view"])
def test_decode_swiglu_fuses_only_when_nothing_else_reads_its_parts(plant):
    """The fused gate / up / SWIGLU writes neither the f32 products nor the GLU's f32 result."""
    g, _ = layer(N=1)
    glu = next(x for x in g.nodes if x.op == kc.GGML_OP["glu"])
    if plant == "glu_output":
        glu.output = 1
    elif plant == "glu_second_use":
        glu.uses = 2
    elif plant == "gate_second_use":
        glu.src[0].contents.uses = 2
    else:
        glu.src[1].contents.view = 1
    names = plan(g)
    assert "decode_swiglu" not in names and "silu_mul_q8x4f" in names


def test_graphs_off_runs_no_concurrent_groups(reference_matvecs):
    g, _ = layer(N=1)
    names = plan(g, graphs=0)
    assert "[" not in names and names[:4] == ["add_norm_q8_f", "matvec_q4k_q8", "matvec_q4k_q8", "matvec_q6k_q8"]
    assert plan(g, concurrent=0) == names


@pytest.mark.parametrize("N,cfg,mm,quant", [
    (8, {}, "matmul_{}_q8kx8", "quantize_cols_k"),           # batch_k256: per-256 slots, x8 tiles
    (4, {}, "matmul_{}_q8kx4", "quantize_cols_k"),           # four columns: x4
    (8, dict(tile=4), "matmul_{}_q8kx4", "quantize_cols_k"),
    (3, dict(q8k=0), "matmul_{}_q8x4", "quantize_cols"),      # Q8K=0: per-32 slots
    (64, dict(attn_tokens=64), "matmul_{}_q8kx8", "quantize_cols_k"),
])
def test_batch_layer_plans(N, cfg, mm, quant):
    g, _ = layer(N=N)
    k = "q8k" if quant == "quantize_cols_k" else "q8"
    # [ADD +] RMS_NORM + MUL in one workgroup per row: add_norm_q8k_f (per 256) or add_norm_q8_f (per 32)
    norm = ["add_norm_q8k_f"] if k == "q8k" else ["add_norm_q8_f"]
    silu = "silu_mul_q8kf" if k == "q8k" else "silu_mul_q8x4f"
    attn = ["rope_set_rows", "flash_decode_f16" if N <= 8 else "attn_masked"]  # past 8 tokens: the matrix cores
    # from 64 columns (the MFMA matmul) every MUL_MAT runs grouped from its input's fp16 form: q / k / v and
    # gate / up one launch each, o and down with the K split whose second half the next reader adds: the
    # FFN norm takes o's along, the layer's last ADD (no norm follows in this one-layer graph) adds down's
    # with one more vector_add first
    qkv = ["matmul_group"] if N >= 64 else ["[", mm.format("q4k"), mm.format("q4k"), mm.format("q6k"), "]"]
    gu = ["matmul_group"] if N >= 64 else ["[", mm.format("q4k"), mm.format("q4k"), "]"]
    o, down = (["matmul_group"], ["matmul_group", "vector_add"]) if N >= 64 else ([mm.format("q4k")], [mm.format("q6k")])
    want = (norm + qkv + attn + [quant] + o + norm + gu + [silu] + down + ["vector_add"])
    assert plan(g, **cfg) == want


def test_batch_groups_on_the_matrix_cores_take_one_grouped_launch(reference_matvecs):
    """The grouped launch is a fusion beyond the reference's (ggml_extra_fusions = 1 restores its
    concurrent group of one by-name matmul per MUL_MAT); below 64 columns, or with per-32 slots, the
    MUL_MATs stay by-name matmuls."""
    g, _ = layer(N=64)
    names = plan(g, attn_tokens=64)
    assert "matmul_group" not in names and names.count("[") == 2
    kc.set_option("ggml_extra_fusions", 0)
    assert plan(g, attn_tokens=64, q8k=0).count("matmul_group") == 0
    assert plan(layer(N=63)[0], attn_tokens=64).count("matmul_group") == 0
    assert plan(g, attn_tokens=64).count("matmul_group") == 4  # q / k / v, o, gate / up, down


@pytest.mark.parametrize("plant", ["second_use", "output", "view"])
def test_second_k_half_is_added_at_once_unless_the_add_alone_reads_the_product(plant):
    """A batch product whose K is split leaves its second half for its one reader, the ADD, whose
    fused norm adds it; a product read twice, a graph output or a view is completed right after its
    matmul."""
    g, t = layer(N=64)
    if plant == "second_use":
        t["o"].uses = 2
    elif plant == "output":
        t["o"].output = 1
    else:
        t["o"].view = 1
    names = plan(g, attn_tokens=64)
    i = names.index("attn_masked")
    assert names[i + 1:i + 5] == ["quantize_cols_k", "matmul_group", "vector_add", "add_norm_q8k_f"], names


def test_masked_batch_attention_is_claimed_past_the_score_limit():
    """A prompt whose score matrix would pass 2^24 values (32 heads x 1024 tokens x 1024 keys: BASELINE
    config 5's prompt) is claimed when it runs on the masked matrix-core kernel, which keeps no scores;
    without a mask (the four fa_* kernels and their score scratch) it is not."""
    s = gg.LayerShape(n_embd=4096, n_head=32, n_head_kv=8, n_ff=1024, head_dim=128, kv_size=1024, neox=True,
                      qk_norm=True)
    g = gg.Graph()
    gg.llama_layer(g, s, 1024, 1024)
    names = kc.ggml_graph_plan(g.nodes, attn_tokens=1024)[0]
    assert "attn_masked" in names
    fa = next(x for x in g.nodes if x.op == kc.GGML_OP["flash_attn_ext"])
    assert kc.ggml_supports_op(fa, attn_tokens=1024)
    fa.src[3] = None
    assert not kc.ggml_supports_op(fa, attn_tokens=1024)


@pytest.mark.parametrize("plant", [None, "norm_second_use", "other_eps", "rope_source"])
def test_per_head_norms_enter_the_attention_only_when_they_feed_its_ropes(plant):
    """Qwen3's per-head q / k RMS_NORM + MUL run in the one-token attention's prologue only when each
    norm is read by its MUL alone, both take one eps, and the ROPEs read those MUL results."""
    s = gg.LayerShape(n_embd=1024, n_head=8, n_head_kv=2, head_dim=128, neox=True, qk_norm=True)
    g, t = gg.Graph(), None
    t = gg.llama_layer(g, s, 1, 90)
    norms = [x for x in g.nodes if x.op == kc.GGML_OP["rms_norm"] and x.ne[0] == 128]
    if plant == "norm_second_use":
        norms[0].uses = 2
    elif plant == "other_eps":
        norms[1].op_params[0] = norms[1].op_params[0] + 1
    elif plant == "rope_source":
        rope = next(x for x in g.nodes if x.op == kc.GGML_OP["rope"])
        rope.src[0] = C.pointer(g.leaf("f32", [128, 8, 1]))
    names = plan(g)
    if plant is None:
        assert names[:2] == ["decode_norm_matvec", "norm_rope_flash_decode_q8"], names
    else:
        assert "norm_rope_flash_decode_q8" not in names and "rms_norm" in names, names


def test_matvec_cols_runs_one_matvec_per_column():
    g, _ = layer(N=3)
    names = plan(g, matvec_cols=1)
    assert names[:1] == ["add_norm_q8_f"]  # not batch_k256: per-32 slots
    assert names[1:11] == ["["] + ["matvec_q4k_q8"] * 6 + ["matvec_q6k_q8"] * 3
    assert "quantize_cols" in names  # the attention output: contiguous columns, one launch


def test_residual_add_fuses_into_the_next_layers_norm():
    g = gg.Graph()
    s = gg.LayerShape()
    t = gg.llama_layer(g, s, 1, 41)
    t["out"].output = 0
    norm = g.rms_norm(t["out"], s.eps)
    cur = g.mul(norm, t["attn_norm"])
    g.mul_mat(t["wq"], cur)
    g.finish()
    names = plan(g)
    # the residual ADD fused with the next layer's norm, whose slots the MUL_MAT takes (no quantizer)
    assert names[-2:] == ["add_norm_q8_f", "matvec_q4k_q8"] and "vector_add" not in names


def norm_mul_graph(n=512, rows=1, weight_rows=1, mm=True):
    g = gg.Graph()
    x = g.leaf("f32", [n, rows])
    w = g.leaf("f32", [n, weight_rows], buffer="weights")
    norm = g.rms_norm(x, 1e-5)
    mul = g.mul(norm, w)
    if mm:
        g.mul_mat(g.leaf("q4k", [n, 64], buffer="weights"), mul)
    return g, norm, mul


def test_norm_mul_fuses():
    g, _, _ = norm_mul_graph()
    g.finish()
    assert plan(g) == ["add_norm_q8_f", "matvec_q4k_q8"]
    g, _, _ = norm_mul_graph(n=8448)  # rows past 8192 values: the reference's two kernels
    g.finish()
    assert plan(g) == ["sumsq_part", "norm_mul_q8_f", "matvec_q4k_q8"]


@pytest.mark.parametrize("plant", ["second_use", "output", "view"])
def test_norm_that_cannot_fuse_runs_alone(plant):
    g, norm, mul = norm_mul_graph()
    if plant == "second_use":
        g.add(norm, norm)
    g.finish()
    if plant == "output":
        norm.output = 1
    if plant == "view":
        norm.view = 1
    names = plan(g)
    # one-pass rms_norm without a weight, the MUL on its own, the MUL_MAT quantizes its input
    assert names[:4] == ["rms_norm", "mul_rows", "quantize_q8x4", "matvec_q4k_q8"]


def test_mul_by_a_matrix_is_not_the_norm_weight():
    g, _, _ = norm_mul_graph(rows=2, weight_rows=2)
    g.finish()
    assert plan(g) == ["rms_norm", "mul_rows", "quantize_cols_k", "matmul_q4k_q8kx4"]


def test_rows_not_a_multiple_of_256_take_the_weighted_rms_norm():
    g, _, _ = norm_mul_graph(n=384, mm=False)
    g.finish()
    assert plan(g) == ["rms_norm"]  # RMS_NORM + MUL as one rms_norm with the weight


def test_add_whose_result_the_norm_does_not_read():
    g = gg.Graph()
    a, b, x = (g.leaf("f32", [512, 1]) for _ in range(3))
    g.add(a, b)
    norm = g.rms_norm(x, 1e-5)
    g.mul(norm, g.leaf("f32", [512], buffer="weights"))
    g.finish()
    assert plan(g) == ["vector_add", "add_norm_q8_f"]


def test_nodes_without_work_are_skipped():
    g, t = layer(N=1)
    t["o"].compute = 0  # not computed by this backend (the scheduler's flag)
    names = plan(g)
    assert "matvec_q4k_q8" not in names and "quantize_q8x4" not in names  # q / k / v fused, o skipped
    kc.set_option("ggml_extra_fusions", 1)
    try:
        names = plan(g)
    finally:
        kc.set_option("ggml_extra_fusions", 0)
    assert names.count("matvec_q4k_q8") == 4 and "quantize_q8x4" not in names
    g = gg.Graph()
    x = g.leaf("f32", [512, 0])
    g.add(x, x)
    g.finish()
    assert plan(g) == []  # an empty node


def test_swiglu_unfused_when_rows_are_not_a_multiple_of_256():
    g = gg.Graph()
    a, b = g.leaf("f32", [96, 3]), g.leaf("f32", [96, 3])
    g.swiglu(a, b)
    g.finish()
    assert plan(g) == ["silu_mul"]


def test_decode_attention_is_split_over_the_context():
    g, _ = layer(N=1, n_kv=20000, kv_size=20480)
    names, ints = kc.ggml_graph_plan(g.nodes)
    assert "rope_flash_decode_q8" in names
    assert ints >= 8 * 313 * 66  # the partials of 8 heads x 313 chunks x (64 values + max + sum)


def test_batch_attention_runs_masked_on_the_matrix_cores():
    g, _ = layer(N=12, n_kv=20000, kv_size=20480)
    names, ints = kc.ggml_graph_plan(g.nodes, attn_tokens=16)
    i = names.index("rope_set_rows")
    assert names[i + 1] == "attn_masked" and "fa_scores" not in names
    assert ints < 8 * 12 * 20000  # no score matrix in the scratch


def test_long_context_batch_attention_takes_the_four_kernels():
    # head_dim 96: not one the masked matrix-core kernel takes; past 16384 keys: the reference's four
    g, _ = layer(N=12, n_kv=20000, kv_size=20480, n_embd=768, head_dim=96)
    names, ints = kc.ggml_graph_plan(g.nodes, attn_tokens=16)
    i = names.index("rope_set_rows")
    assert names[i:i + 5] == ["rope_set_rows", "fa_scores", "fa_max", "fa_exp", "fa_values"]
    assert ints >= 8 * 12 * 20000  # the scores of 8 heads x 12 tokens in the scratch


def test_fused_producers_beyond_their_limit_run_unfused():
    g, _, _ = norm_mul_graph(n=4096, rows=4096, mm=False)
    g.finish()
    assert plan(g, attn_tokens=8) == ["rms_norm"]
    g = gg.Graph()
    a, b = g.leaf("f32", [8192, 2048]), g.leaf("f32", [8192, 2048])
    g.swiglu(a, b)
    g.finish()
    assert plan(g) == ["silu_mul"]


def test_unsupported_nodes_are_refused_before_any_launch():
    g, t = layer(N=1)
    t["wq"].buffer = kc.GGML_BUFFER["other"]  # a weight outside this backend's buffers
    with pytest.raises(kc.KcError) as e:
        plan(g)
    assert e.value.name == "UnsupportedOperation" and "node 2" in str(e.value)
    g = gg.Graph()
    x = g.leaf("f32", [64])
    g.node("other", "f32", [64], [x])
    with pytest.raises(kc.KcError) as e:
        plan(g)
    assert e.value.name == "UnsupportedOperation"


def test_disabled_claims_nothing_and_makes_no_backend():
    g, t = layer(N=1)
    assert not kc.ggml_supports_op(t["q"], disabled=1)
    assert not kc.ggml_offers_kv_buffer(disabled=1)
    with pytest.raises(kc.KcError) as e:
        kc.GgmlBackend(disabled=1)
    assert e.value.name == "UnsupportedOperation"


def test_scratch_requirement(reference_matvecs):
    g, _ = layer(N=1)
    # four per-32 slots of 512 or 1024 values (11 ints per 32: 880), the attention partials of 8 heads x
    # 1 chunk x (64 values + max + sum) = 528
    assert kc.ggml_graph_plan(g.nodes)[1] == 880 + 528


def test_scratch_requirement_of_the_fused_decode_layer():
    g, _ = layer(N=1)
    # the norms run inside the matvec launches: the slots of the attention output (512 values: 176) and
    # of the SWIGLU result (1024: 352), and the attention partials (528)
    assert kc.ggml_graph_plan(g.nodes)[1] == 176 + 352 + 528


# ---- supports_op ---------------------------------------------------------------------------------------------

def test_layer_nodes_are_all_claimed():
    for N, cfg in [(1, {}), (8, {}), (64, dict(attn_tokens=64))]:
        g, _ = layer(N=N)
        assert all(kc.ggml_supports_op(n, **cfg) for n in g.nodes)


def test_attention_of_batches_beyond_attn_tokens_is_not_claimed():
    g, t = layer(N=9)
    assert not kc.ggml_supports_op(t["attn"])
    assert kc.ggml_supports_op(t["attn"], attn_tokens=9)
    assert kc.ggml_supports_op(t["q"])  # MUL_MAT: any batch


def test_matmul_only_and_attn_switches():
    g, t = layer(N=1)
    assert kc.ggml_supports_op(t["q"], matmul_only=1) and not kc.ggml_supports_op(t["norm"], matmul_only=1)
    assert not kc.ggml_supports_op(t["k_set"], attn=0) and not kc.ggml_supports_op(t["attn"], attn=0)
    assert kc.ggml_supports_op(t["rope"] if "rope" in t else t["qr"], attn=0)
    assert not kc.ggml_offers_kv_buffer(attn=0) and not kc.ggml_offers_kv_buffer(matmul_only=1)
    assert kc.ggml_offers_kv_buffer()


def mm_case(wtype="q4k", k=512, rows=64, ncols=3, buffer="weights", **plant):
    g = gg.Graph()
    w = g.leaf(wtype, [k, rows], buffer=buffer)
    x = g.leaf("f32", [k, ncols])
    for f, v in plant.items():
        if f == "w_ne2":
            w.ne[2] = v
        elif f == "x_nb1":
            x.nb[1] = v
        elif f == "x_ne0":
            x.ne[0] = v
    return g.mul_mat(w, x)


@pytest.mark.parametrize("case,want", [
    (dict(), True), (dict(wtype="q6k"), True), (dict(wtype="f16", k=514), True),
    (dict(buffer="other"), False),      # the weight must be in this backend's (repacked) buffers
    (dict(k=300), False),               # K-quant k % 256
    (dict(rows=60), False),             # rows % 8
    (dict(wtype="f16", k=513), False),  # fp16 k even
    (dict(w_ne2=2), False),             # 2-D weights only
    (dict(x_nb1=4 * 600), False),       # the input contiguous
    (dict(x_ne0=256), False),           # the input's rows as long as the weight's
])
def test_mul_mat_rules(case, want):
    assert kc.ggml_supports_op(mm_case(**case)) == want


def rope_case(**plant):
    g = gg.Graph()
    x = g.leaf("f32", [64, 8, 3])
    pos = g.leaf("i32", [3])
    ff = g.leaf("f32", [32]) if plant.pop("ff", False) else None
    kw = dict(neox=plant.pop("neox", False), ff=ff)
    for k in ("freq_scale", "ext_factor", "attn_factor", "p15"):
        if k in plant:
            kw[k] = plant.pop(k)
    n_dims = plant.pop("n_dims", 64)
    if plant.pop("pos_i64", False):
        pos = g.leaf("i64", [3])
    t = g.rope(x, pos, n_dims, freq_base=10000.0, **kw)
    if plant.pop("mode", None) is not None:
        t.op_params[2] = 8  # another rope mode (e.g. multi-section)
    return t


@pytest.mark.parametrize("case,want", [
    (dict(), True), (dict(neox=True), True), (dict(ff=True), True),
    (dict(n_dims=32), False),           # partial rotation
    (dict(freq_scale=0.5), False), (dict(ext_factor=1.0), False), (dict(attn_factor=2.0), False),
    (dict(p15=1), False), (dict(mode=8), False), (dict(pos_i64=True), False),
])
def test_rope_rules(case, want):
    assert kc.ggml_supports_op(rope_case(**case)) == want


def test_elementwise_rules():
    g = gg.Graph()
    a, b = g.leaf("f32", [512, 2]), g.leaf("f32", [512, 2])
    row = g.leaf("f32", [512])
    odd = g.leaf("f32", [12, 1])
    assert kc.ggml_supports_op(g.add(a, b)) and kc.ggml_supports_op(g.mul(a, row)) and kc.ggml_supports_op(g.mul(a, b))
    assert not kc.ggml_supports_op(g.add(a, row))  # ADD: same shapes only
    assert not kc.ggml_supports_op(g.mul(odd, odd))  # 12 values: not a multiple of 8
    assert kc.ggml_supports_op(g.rms_norm(a, 1e-6))
    f16 = g.leaf("f16", [512, 2])
    assert not kc.ggml_supports_op(g.rms_norm(f16, 1e-6))
    assert kc.ggml_supports_op(g.swiglu(a, b)) and not kc.ggml_supports_op(g.swiglu(a, b, op=1))
    assert not kc.ggml_supports_op(g.swiglu(a, b, swapped=1))


def test_set_rows_and_attention_rules():
    g, t = layer(N=2)
    assert kc.ggml_supports_op(t["k_set"]) and kc.ggml_supports_op(t["attn"])
    t["k_cache"].buffer = t["k_set"].buffer = kc.GGML_BUFFER["other"]
    assert not kc.ggml_supports_op(t["k_set"])  # not a KV buffer of this backend
    t["k_view"].buffer = kc.GGML_BUFFER["other"]
    assert not kc.ggml_supports_op(t["attn"])
    g, t = layer(N=2)
    t["attn"].op_params[2] = gg.f32bits(30.0)  # logit softcap
    assert not kc.ggml_supports_op(t["attn"])
    g, t = layer(N=2)
    t["mask"].type = kc.GGML_TYPE["f32"]
    assert not kc.ggml_supports_op(t["attn"])


def test_host_environment_switches(monkeypatch):
    for v in ("DISABLE", "MATMUL_ONLY", "ATTN", "ATTN_TOKENS", "CONCURRENT", "GRAPHS", "MATVEC_COLS", "Q8K", "TILE",
              "ROW_BLOCK", "PROFILE"):
        monkeypatch.delenv(f"GGML_KERNELCORE_{v}", raising=False)
    assert kc.ggml_config_dict(kc.ggml_config()) == dict(matvec_cols=0, q8k=1, tile=8, row_block=8, disabled=0,
                                                         matmul_only=0, attn=1, attn_tokens=8, concurrent=1, graphs=1,
                                                         profile=0)
    monkeypatch.setenv("GGML_KERNELCORE_ATTN_TOKENS", "-3")
    monkeypatch.setenv("GGML_KERNELCORE_GRAPHS", "0")
    monkeypatch.setenv("GGML_KERNELCORE_DISABLE", "yes")  # only "1" disables
    monkeypatch.setenv("GGML_KERNELCORE_TILE", "4")
    monkeypatch.setenv("GGML_KERNELCORE_PROFILE", "2")  # "1" or "2" (ggml-kernelcore.cpp:1033-1035)
    d = kc.ggml_config_dict(kc.ggml_config())
    assert (d["attn_tokens"], d["graphs"], d["disabled"], d["tile"], d["profile"]) == (0, 0, 0, 4, 2)
    monkeypatch.setenv("GGML_KERNELCORE_PROFILE", "3")
    assert kc.ggml_config_dict(kc.ggml_config())["profile"] == 0


# ---- graphs whose tensors share memory as ggml's allocator places them --------------------------------------

def shared_layer(N=1, outputs=(), inplace_views=True, **kw):
    """The layer graph with its computed nodes placed by gg.share_memory (one fake arena); names in
    `outputs` are marked graph outputs before the placement (as llama.cpp flags them)."""
    g = gg.Graph()
    t = gg.llama_layer(g, gg.LayerShape(**kw), N, 40 + N)
    for name in outputs:
        t[name].output = 1
    gg.share_memory(g, lambda n: 1 << 24, inplace_views=inplace_views)
    return g, t


def spans(t):
    end = 4 + sum((t.ne[d] - 1) * t.nb[d] for d in range(4))
    return t.data, t.data + end


@pytest.mark.parametrize("inplace_views", [True, False])
@pytest.mark.parametrize("N", [1, 8, 64])
def test_shared_memory_never_overlaps_two_live_tensors(N, inplace_views):
    """The placement itself: a computed node's memory is not overlapped by any other computed
    non-view node between the first's definition and its last reader (views counted as readers of
    their base), unless the second is the first's in-place successor (same address, defined by an
    op that reads it last); in-place placement happens (RMS_NORM + MUL, the residual ADD) and memory
    is reused (the arena is smaller than the nodes' sum)."""
    g, t = shared_layer(N=N, inplace_views=inplace_views)
    base = lambda x: g.view_of.get(id(x), (x, 0))[0]
    nodes = [x for x in g.nodes]
    last = {}
    for i, x in enumerate(nodes):
        for s in g.srcs[id(x)]:
            last[id(base(s))] = i
    own = [(i, x) for i, x in enumerate(nodes) if not x.view]
    for a_i, a in own:
        end = max(last.get(id(a), a_i), a_i) if not a.output else len(nodes)
        for b_i, b in own:
            if b_i <= a_i or b_i > end:
                continue
            lo_a, hi_a = spans(a)
            lo_b, hi_b = spans(b)
            if lo_a < hi_b and lo_b < hi_a:  # only an in-place successor reading a last
                assert b.data == a.data and kc_name(b) in gg.INPLACE_OPS and b_i == last[id(a)], (a_i, b_i)
    assert t["cur"].data == t["norm"].data  # MUL in place over RMS_NORM
    assert t["out"].data == t["down"].data  # the residual ADD in place over the down product
    assert (t["qr"].data == t["q"].data) == inplace_views  # ROPE over the reshaped q


def kc_name(x):
    return gg.kc_op_name(x)


def test_shared_memory_puts_the_attention_output_on_the_dead_norm_output():
    """ggml's best fit: a prompt's FLASH_ATTN_EXT output ([D, H, N] f32, the size of the normed
    activations the q / k / v products read) takes the block the attention norm's output left: the
    aliasing under which a MUL_MAT input cache keyed by address hands the o projection the normed
    activations' 8-bit slots. The plan keys the cache by tensor: o quantizes its own input."""
    g, t = shared_layer(N=64)
    assert t["attn"].data == t["cur"].data
    names = plan(g, attn_tokens=64)
    # cur (per 256, MFMA form) for q / k / v, then the attention output quantized for o
    assert names.count("quantize_cols_k") == 1 and names.index("quantize_cols_k") > names.index("attn_masked")


def test_fused_attention_writes_no_dead_intermediates_and_refuses_live_aliased_ones():
    """One token with in-place ROPE (qr on q's memory, kr on k's): nothing outside the fused launch reads
    qr or kr, so the fusion stands (it writes neither). Marked graph outputs, qr / kr must be written,
    and their chunk-0 writes would race with the other chunks' reads of q / k: the fusion is refused
    and the nodes run as rope_set_rows + flash_decode_q8 (both element by element in place)."""
    g, t = shared_layer(N=1)
    assert t["qr"].data == t["q"].data and t["kr"].data == t["k"].data
    assert "rope_flash_decode_q8" in plan(g)
    g, t = shared_layer(N=1, outputs=("qr",))
    names = plan(g)
    assert "rope_flash_decode_q8" not in names and "rope_set_rows" in names and "flash_decode_q8" in names
    g, t = shared_layer(N=1, outputs=("qr",), inplace_views=False)  # written, not aliased: fused
    assert t["qr"].data != t["q"].data and "rope_flash_decode_q8" in plan(g)


def test_fused_qk_norm_attention_refuses_live_aliased_norm_outputs():
    kw = dict(n_embd=1024, n_head=8, n_head_kv=2, head_dim=128, neox=True, qk_norm=True)
    g, t = shared_layer(N=1, **kw)
    assert t["qn"].data == t["q"].data  # RMS_NORM over the reshaped q, MUL over that, ROPE over that
    assert "norm_rope_flash_decode_q8" in plan(g)
    g, t = shared_layer(N=1, outputs=("qn",), **kw)
    assert "norm_rope_flash_decode_q8" not in plan(g)


def test_add_of_a_pending_product_with_itself_completes_the_product_first():
    """ADD(y, y) of a K-split batch product y: both operands need y's second K half, so it is added to
    y (vector_add) before the fused ADD + norm reads y twice. ggml counts one use per src slot (y has
    two), which keeps y from being left pending; forced to one use, the walk still completes y first."""
    g = gg.Graph()
    x = g.leaf("f32", [512, 64])
    y = g.mul_mat(g.leaf("q4k", [512, 512], buffer="weights"), x)
    a = g.add(y, y)
    cur = g.mul(g.rms_norm(a, 1e-5), g.leaf("f32", [512], buffer="weights"))
    g.mul_mat(g.leaf("q4k", [512, 256], buffer="weights"), cur)
    g.finish()
    # (the last product's K is split too; nothing reads it, so the walk's end completes it)
    want = ["quantize_cols_k", "matmul_group", "vector_add", "add_norm_q8k_f", "matmul_group", "vector_add"]
    assert y.uses == 2 and plan(g) == want
    y.uses = 1
    assert plan(g) == want

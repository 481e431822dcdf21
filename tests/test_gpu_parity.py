"""GPU parity of the HIP path (through the C ABI / Kernels) against the CPU oracle.

Bars:
  * integer work (quantizer output, dequantized weights): bit-exact;
  * outputs: max|y - ref| <= 1e-2 * ||ref||_inf against the fp32-dequant, double-accumulated
    oracle (bench/bench_w4a16.cu:94-103, 120) -- and much tighter bounds where the arithmetic
    allows it (noted per test).
"""
import numpy as np
import pytest
import torch

from nanoserve_amd import synth
from tests.conftest import to_dev, to_host_bits

pytestmark = pytest.mark.gpu

TOL = 1e-2  # max|err| <= TOL * ||ref||_inf


def run_linear(kernels, X, Wq, S, G):
    y = kernels.w4_linear(to_dev(X, torch.bfloat16), to_dev(Wq, torch.int32),
                          to_dev(S, torch.bfloat16), G)
    torch.cuda.synchronize()
    return synth.bf16_bits_to_f32(to_host_bits(y)).astype(np.float64)


def check_close(oracle, y, ref, tight=None):
    err = oracle.max_rel_err(y, ref)
    assert err <= TOL, err
    if tight is not None:
        assert err <= tight, err
    return err


def check_bf16_faithful(y, ref, rel_slack):
    """y is bf16(RNE) of a value within rel_slack * ||ref||_inf of ref: |y - ref| <= half a
    bf16 ulp of ref plus that slack."""
    bound = np.abs(ref) * 2.0 ** -8 + rel_slack * np.max(np.abs(ref))
    assert np.all(np.abs(y - ref) <= bound), float(np.max(np.abs(y - ref) - bound))


# ----------------------------------------------------------------- reference correctness case
@pytest.fixture(scope="module")
def ref_case(oracle):
    N, K, G, Mmax = 256, 512, 128, 128
    W = oracle.hash_fill(N * K, 11, 0.05).reshape(N, K)
    X = oracle.hash_fill(Mmax * K, 12, 1.0).reshape(Mmax, K)
    Wq, S = oracle.quantize(W, G)
    return dict(N=N, K=K, G=G, W=W, X=X, Wq=Wq, S=S, ref=oracle.linear_f64(X, Wq, S, G))


def test_reference_case_quantize_bitexact(kernels, ref_case):
    Wq, S = kernels.w4_quantize(to_dev(ref_case["W"], torch.bfloat16), ref_case["G"])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host_bits(Wq), ref_case["Wq"])
    np.testing.assert_array_equal(to_host_bits(S), ref_case["S"])


@pytest.mark.parametrize("M", [1, 8, 128])
def test_reference_case_linear(kernels, oracle, ref_case, M):
    c = ref_case
    y = run_linear(kernels, c["X"][:M], c["Wq"], c["S"], c["G"])
    ref = c["ref"][:M]
    if M <= 8:   # exact dequant, fp32 accumulation: only the bf16 output rounding remains
        check_bf16_faithful(y, ref, 1e-5)
    else:        # GEMM stages weights as bf16 (reference semantics): ~2e-3 like the reference
        check_close(oracle, y, ref, tight=5e-3)
        staged = oracle.linear_f64(c["X"][:M], c["Wq"], c["S"], c["G"], bf16_weights=True)
        check_bf16_faithful(y, staged, 1e-5)


# ----------------------------------------------------------------- bit-exact dequant probes
def _onehot_probe(kernels, oracle, N, K, G, M, staged, seed, ks=None, call=None):
    """X rows are unit vectors e_k, so y[m][n] = w[n][k_m] with no rounding but the bf16 output:
    y must equal bf16_rne of the (exact or bf16-staged) dequantized weight, bit for bit.
    ``ks``: the k probed (default every k); ``call(x, Wq, S)``: the entry point (default
    w4_linear)."""
    Wq, S = synth.weights(N, K, G, seed=seed)
    Wq[0, :] = 0x00000000            # q = 0 -> -8 everywhere in row 0
    Wq[1, :] = 0xFFFFFFFF            # q = 15 -> 7 everywhere in row 1
    deq = oracle.dequant_bf16(Wq, S, G) if staged else oracle.f32_to_bf16(oracle.dequant_f32(Wq, S, G))
    wq_d, s_d = to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    call = call or (lambda x, w, sc: kernels.w4_linear(x, w, sc, G))
    ks = list(range(K)) if ks is None else list(ks)
    for i0 in range(0, len(ks), M):
        kk = ks[i0:i0 + M]
        X = np.zeros((M, K), dtype=np.uint16)
        for m, k in enumerate(kk):
            X[m, k] = 0x3F80          # 1.0
        y = call(to_dev(X, torch.bfloat16), wq_d, s_d)
        torch.cuda.synchronize()
        got = to_host_bits(y).reshape(M, -1)
        for m, k in enumerate(kk):
            np.testing.assert_array_equal(got[m], deq[:, k], err_msg=f"k={k}")


@pytest.mark.parametrize("G", [128, 256])
def test_gemv_dequant_bitexact(kernels, oracle, G):
    _onehot_probe(kernels, oracle, N=80, K=512, G=G, M=8, staged=False, seed=G)


# M = 1 layouts of w4_gemv_m1_kernel (the launcher picks them from N and K on the device's CU
# count): the one-round layout (N = 80, K = 512), seven-wave persistent 16-row groups with the
# activation fragments held in registers (gate/up-like, N = 16400, K = 1792), eight-row groups
# (N = 8000, K = 4096) and sixteen-wave workgroups for long rows (K = 8192). Long rows are
# probed at every k of their first and last 256 and at a seeded sample in between, which covers
# every nibble, word, piece and block position.
M1_PROBES = [(80, 512), (16400, 1792), (8000, 4096), (64, 8192)]


def _m1_probe_ks(K, seed):
    if K <= 2048:
        return range(K)
    mid = np.random.default_rng(seed).choice(np.arange(256, K - 256), 256, replace=False)
    return sorted(set(range(256)) | set(range(K - 256, K)) | set(int(k) for k in mid))


@pytest.mark.parametrize("N,K", M1_PROBES)
def test_gemv_m1_dequant_bitexact(kernels, oracle, N, K):
    """The M = 1 kernel (ns_w4_linear at M = 1) returns each dequantized weight bit for bit."""
    _onehot_probe(kernels, oracle, N=N, K=K, G=128, M=1, staged=False, seed=N + K,
                  ks=_m1_probe_ks(K, N))


@pytest.mark.parametrize("N,K", M1_PROBES)
def test_gemv_decode_dequant_bitexact(kernels, oracle, N, K):
    """The fused decode GEMV (ns_w4_gemv_decode with a plain activation: no norm, no SwiGLU)
    returns each dequantized weight bit for bit on the same layouts."""
    _onehot_probe(kernels, oracle, N=N, K=K, G=128, M=1, staged=False, seed=N + K + 1,
                  ks=_m1_probe_ks(K, N + 1),
                  call=lambda x, w, sc: kernels.gemv_decode(w, sc, 128, x=x[0]))


def test_gemv_generic_dequant_bitexact(kernels, oracle):
    _onehot_probe(kernels, oracle, N=48, K=96, G=32, M=8, staged=False, seed=2)


def test_gemm_dequant_bitexact(kernels, oracle):
    _onehot_probe(kernels, oracle, N=256, K=512, G=128, M=128, staged=True, seed=5)


# ----------------------------------------------------------------- benchmark configurations
CONFIG_SHAPES = [synth.QWEN15B_GATE] + list(synth.QWEN7B_LAYERS)


@pytest.mark.parametrize("name,N,K", CONFIG_SHAPES, ids=[s[0] for s in CONFIG_SHAPES])
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_gemv_configs(kernels, oracle, name, N, K, M):
    """Every config shape at M = 1, 2, 4 and 8 (the M = 2..8 planner picks its group height and
    workgroups per CU per shape and M)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + K)
    X = synth.activations(M, K, seed=100, per_row_seed=True)
    y = run_linear(kernels, X, Wq, S, G)
    ref = oracle.linear_f64(X, Wq, S, G)
    check_close(oracle, y, ref, tight=2.0 ** -8)   # bf16 output: half an ulp is <= 2^-8 |y|
    check_bf16_faithful(y, ref, 2e-5)


@pytest.mark.parametrize("N,K,Ms", [(200, 12544, (2, 5, 8)), (3584, 18944, (3, 6, 7)),
                                    (1000, 20480, (2, 8)), (4104, 16384, (4, 8)),
                                    (1536, 8960, (2, 8)), (264, 8448, (3, 8))])
def test_gemv_ksplit(kernels, oracle, N, K, Ms):
    """M = 2..8 at K of more than 32 pairs (256 k each): through ns_w4_linear_ws the kernel runs
    in two or three K slices whose fp32 partials a merge launch sums, through ns_w4_linear in one
    pass. Both within half a bf16 ulp (+2e-5 ||ref||) of the oracle, every M listed, ragged N
    (row groups cut by N), and each call repeated bit for bit after calls of other shapes (the
    workspace reused; ns_w4_linear keeps nothing between calls)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 3 * K)
    wd, sd = to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    work = kernels.w4_linear_workspace(max(Ms), N, K, G)
    assert work is not None and work.numel() == -(-K // 8192) * max(Ms) * N * 4
    first = {}
    for M in Ms:
        X = synth.activations(M, K, seed=M + 40, per_row_seed=True)
        xd = to_dev(X, torch.bfloat16)
        ref = oracle.linear_f64(X, Wq, S, G)
        for w in (work, None):
            y = kernels.w4_linear(xd, wd, sd, G, work=w)
            torch.cuda.synchronize()
            check_bf16_faithful(synth.bf16_bits_to_f32(to_host_bits(y)).astype(np.float64), ref,
                                2e-5)
            first[(M, w is None)] = (xd, to_host_bits(y))
    for (M, unsplit), (xd, bits) in reversed(list(first.items())):
        y = kernels.w4_linear(xd, wd, sd, G, work=None if unsplit else work)
        np.testing.assert_array_equal(to_host_bits(y), bits)


def test_gemv_linear_ws_rejects(kernels):
    """ns_w4_linear_ws needs a workspace of ns_w4_linear_workspace bytes where the shape splits,
    and takes none where it does not (the call is then ns_w4_linear)."""
    lib = kernels.lib
    assert lib.ns_w4_linear_workspace(8, 3584, 18944, 128) == 3 * 8 * 3584 * 4
    assert lib.ns_w4_linear_workspace(8, 3584, 8192, 128) == 0      # 32 pairs: one pass
    assert lib.ns_w4_linear_workspace(1, 3584, 18944, 128) == 0     # M = 1
    assert lib.ns_w4_linear_workspace(128, 3584, 18944, 128) == 0   # GEMM
    x = torch.zeros(8, 18944, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(64, 18944 // 8, dtype=torch.int32, device="cuda")
    s = torch.zeros(64, 148, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(8, 64, dtype=torch.bfloat16, device="cuda")
    need = lib.ns_w4_linear_workspace(8, 64, 18944, 128)
    work = torch.zeros(need, dtype=torch.uint8, device="cuda")
    args = (x.data_ptr(), w.data_ptr(), s.data_ptr(), y.data_ptr(), 8, 64, 18944, 128)
    assert lib.ns_w4_linear_ws(*args, None, 0, None) == -2
    assert lib.ns_w4_linear_ws(*args, work.data_ptr(), need - 4, None) == -2
    assert lib.ns_w4_linear_ws(*args, work.data_ptr() + 4, need - 4, None) == -2
    assert lib.ns_w4_linear_ws(*args, work.data_ptr(), need, None) == 0
    small = (x.data_ptr(), w.data_ptr(), s.data_ptr(), y.data_ptr(), 8, 64, 2048, 128)
    assert lib.ns_w4_linear_ws(*small, None, 0, None) == 0
    torch.cuda.synchronize()


def test_gemv_ksplit_graph(kernels, oracle):
    """The M = 8 GEMV at K = 18944 under graph capture, split (with a workspace) and in one pass
    (ns_w4_linear): on a fresh stream each replay equals the eager call of the same entry
    point bit for bit, with eager calls of other shapes between replays."""
    N, K, G, M = 1024, 18944, 128, 8
    Wq, S = synth.weights(N, K, G, seed=91)
    X = synth.activations(M, K, seed=92, per_row_seed=True)
    ref = oracle.linear_f64(X, Wq, S, G)
    xd, wd, sd = to_dev(X, torch.bfloat16), to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    work = kernels.w4_linear_workspace(M, N, K, G)
    for w in (work, None):
        eager = kernels.w4_linear(xd, wd, sd, G, work=w)
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            y = kernels.w4_linear(xd, wd, sd, G, work=w)
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            got = synth.bf16_bits_to_f32(to_host_bits(y)).astype(np.float64)
            check_bf16_faithful(got, ref, 2e-5)
            assert torch.equal(y, eager)
            kernels.w4_linear(xd[:3], wd, sd, G)
            torch.cuda.synchronize()


# Long rows at M >= 6 with about one 16-row group per compute unit (3/4 to 1 of the CUs; on
# MI355X's 256 CUs, N from 3072 to 4096) run the chunked-activation kernel through both entry
# points: chunks of 4096 k whose last one is partial (K = 8448: 33 pairs, a one-pair last
# chunk; K = 12544: 49 pairs), ragged N (3590: the last tile cut, an odd tile count), and the
# largest K (20480).
M8C_SHAPES = [(3590, 8448, (6, 8)), (3104, 12544, (7,)), (4096, 20480, (8,)), (3584, 18944, (6, 8))]


@pytest.mark.parametrize("N,K,Ms", M8C_SHAPES)
def test_gemv_m8_chunked(kernels, oracle, N, K, Ms):
    """Within half a bf16 ulp (+2e-5 ||ref||) of the oracle; ns_w4_linear and ns_w4_linear_ws
    give the same bits (one kernel, the workspace unused), and a graph replay on a fresh stream
    repeats the eager call bit for bit."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 5 * K)
    wd, sd = to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    work = kernels.w4_linear_workspace(max(Ms), N, K, G)
    for M in Ms:
        X = synth.activations(M, K, seed=M + 50, per_row_seed=True)
        xd = to_dev(X, torch.bfloat16)
        ref = oracle.linear_f64(X, Wq, S, G)
        y = kernels.w4_linear(xd, wd, sd, G)
        yw = kernels.w4_linear(xd, wd, sd, G, work=work)
        torch.cuda.synchronize()
        check_bf16_faithful(synth.bf16_bits_to_f32(to_host_bits(y)).astype(np.float64), ref, 2e-5)
        assert torch.equal(y, yw)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            yg = kernels.w4_linear(xd, wd, sd, G)
        for _ in range(2):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(yg, y)
            kernels.w4_linear(xd[:2], wd, sd, G)
            torch.cuda.synchronize()


def test_gemv_m8_chunked_dequant_bitexact(kernels, oracle):
    """The chunked kernel returns each dequantized weight bit for bit: every k of the first and
    last 256, both sides of each chunk boundary, and a seeded sample in between."""
    N, K = 3584, 8448
    rng = np.random.default_rng(17)
    edge = set(range(256)) | set(range(K - 256, K))
    for b in (4096, 8192):
        edge |= set(range(b - 16, b + 16))
    mid = rng.choice(np.arange(256, K - 256), 96, replace=False)
    _onehot_probe(kernels, oracle, N=N, K=K, G=128, M=8, staged=False, seed=23,
                  ks=sorted(edge | set(int(k) for k in mid)))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6, 7, 8])
def test_gemv_every_m(kernels, oracle, M):
    N, K, G = 200, 1024, 128       # N not a multiple of 16: row-tile tail
    Wq, S = synth.weights(N, K, G, seed=M)
    X = synth.activations(M, K, seed=M + 1)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 1e-5)


@pytest.mark.parametrize("N,K", [(40, 128), (200, 512), (4608, 2048), (16400, 1792), (16400, 4096),
                                 (16400, 7168), (1000, 8192), (64, 16384), (300, 2560)])
def test_gemv_m1_kgroup_counts(kernels, oracle, N, K):
    """M = 1 over k-group counts C = K / 128 for which the launcher does (C in 1, 4, 16, 14, 32, 56,
    64, 128) and does not (C = 20) keep each lane's activation fragments in registers, with each
    of the wave counts the planner picks (8, 14, 16)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N ^ K)
    X = synth.activations(1, K, seed=K + 7)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("N,K", [(4608, 3584), (3584, 3584), (4100, 3584), (4609, 3584), (257, 2560),
                                 (5000, 1024), (8960, 1536), (255, 256), (16384, 512), (12288, 1024),
                                 (20480, 768)])
def test_gemv_m1_one_round_groups(kernels, oracle, N, K):
    """M = 1 shapes small enough for one workgroup per CU with ceil(N / CUs) rows each: row
    groups whose pieces end inside a 1 KiB block (the last block partly another group's), a last
    group shorter than the rest (N tails), (4609, 3584) just past the one-round limit, and short
    rows with more rows per CU than waves (64, 48 and 80 rows on 14, 14 and 16 waves)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N * 3 + K)
    X = synth.activations(1, K, seed=N + 11)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("N,K", [(1536, 8960), (2048, 11008), (100, 8192), (8192, 8192),
                                 (5120, 13824), (3584, 18944), (4100, 18944), (8000, 8192)])
def test_gemv_m1_long_row_layouts(kernels, oracle, N, K):
    """M = 1 with long rows (K / 128 >= 64) in each layout the planner picks on MI355X's 256
    CUs: one round of ceil(N / CUs) rows per CU on sixteen waves when 16-row groups would fill
    half the CUs or fewer (6, 8 and 1 rows), 16-row groups one per CU (224 groups) and over two
    full rounds (512 groups), and one round on fourteen waves between one and two rounds of
    16-row groups (257, 320 and 500 groups: 17, 20 and 32 rows per CU)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 5 * K)
    X = synth.activations(1, K, seed=N + 13)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("N,K", [(2048, 1536), (2560, 2048), (22016, 2048), (17920, 1536),
                                 (8960, 1536), (6144, 4096), (28672, 4096), (5120, 5120),
                                 (4096, 14336)])
def test_gemv_m1_model_layouts(kernels, oracle, N, K):
    """M = 1 layouts the planner picks for layers of other model sizes (on MI355X's 256 CUs):
    eight-wave 16-row groups, two per CU, for tiny layers and for wide ones whose K / 128 is a
    multiple of 8 but not of 7 (2048 x 1536, 2560 x 2048, 22016 x 2048, 28672 x 4096), 16-row
    groups past 512 groups with short rows (17920 x 1536), one round per CU at sixteen or fourteen
    waves (8960 x 1536, 6144 x 4096, 5120 x 5120) and fourteen waves where they fit
    K / 128 = 112 (4096 x 14336)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 7 * K)
    X = synth.activations(1, K, seed=N + 17)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("M,N,K", [(8, 17920, 1536), (2, 17920, 1536), (4, 28672, 4096), (7, 28672, 4096)])
def test_gemv_small_batch_wide_layers(kernels, oracle, M, N, K):
    """M = 2..8 layouts the group planner picks for wide layers beyond the 7B set (on MI355X's 256
    CUs): two workgroups per CU at six waves (1.5B gate/up, 6 pairs), 32-row groups at sixteen
    waves when they fill every CU (Llama-3-8B gate/up, 16 pairs)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + K + M)
    X = synth.activations(M, K, seed=M + 21, per_row_seed=True)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("M", [2, 5, 8])
@pytest.mark.parametrize("N,K", [(24, 256), (200, 4096), (136, 4352), (72, 12288), (40, 16384),
                                 (24, 18944), (9, 20480)])
def test_gemv_small_batch_pair_counts(kernels, oracle, M, N, K):
    """M = 2..8 over 256-k pair counts P = K / 256 that give each of the activation register
    set sizes (1..5 pairs per wave) and wave counts (1, 9, 15, 16) of the half-pair kernel, with
    N tails inside an 8-row tile and inside a two-tile group."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 3 * K + M)
    X = synth.activations(M, K, seed=K + M, per_row_seed=True)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("M", [2, 5, 8])
@pytest.mark.parametrize("N,K", [(200, 384), (300, 1920), (1000, 3712), (72, 3968)])
def test_gemv_small_batch_odd_chunks(kernels, oracle, M, N, K):
    """M = 2..8 with an odd number of 128-k chunks (K not a multiple of 256, up to 32 chunks):
    the kernel that stages each 16-row group's weights in LDS, with 8, 14 and 16 waves."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 7 * K + M)
    X = synth.activations(M, K, seed=K + 2 * M, per_row_seed=True)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("M,N,K", [(8, 3521, 896), (3, 161, 1408), (5, 17, 384), (4, 333, 4224),
                                   (7, 1001, 4480)])
def test_gemv_small_batch_odd_scale_count(kernels, oracle, M, N, K):
    """M = 2..8 where N x K / 128 is odd (odd N, odd chunk count): the kernels that load the scale
    array 16 bytes at a time must still see its last scale, which shares a dword with the two
    bytes after the array (up to 32 chunks: the LDS-staged kernel; beyond, the LDS-activation
    kernel)."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 3 * K + M)
    X = synth.activations(M, K, seed=K + 5 * M, per_row_seed=True)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("M,N,K", [(8, 3521, 896), (4, 333, 4224)])
def test_gemv_small_batch_unaligned_scales(kernels, oracle, M, N, K):
    """The same shapes with the scale array at a 2-byte (not 4-byte) aligned address, as the C ABI
    allows: the launcher takes the kernel with 2-byte scale loads there, so nothing past the
    array is read, and the outputs stay faithful."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + 11 * K + M)
    X = synth.activations(M, K, seed=K + 9 * M, per_row_seed=True)
    C = K // G
    sb = torch.zeros(N * C + 8, dtype=torch.bfloat16, device="cuda")
    s_dev = sb[1:1 + N * C].view(N, C)
    s_dev.copy_(to_dev(S, torch.bfloat16))
    assert s_dev.data_ptr() % 4 == 2
    y = kernels.w4_linear(to_dev(X, torch.bfloat16), to_dev(Wq, torch.int32), s_dev, G)
    torch.cuda.synchronize()
    yh = synth.bf16_bits_to_f32(to_host_bits(y)).astype(np.float64)
    check_bf16_faithful(yh, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("M,N,K", [(3, 4600, 3584), (7, 37880, 3584), (4, 3580, 3584), (6, 3577, 18944),
                                   (8, 9000, 7168)])
def test_gemv_small_batch_group_heights(kernels, oracle, M, N, K):
    """M = 2..8 on the config shapes with N tails: shapes where the half-pair kernel's planner
    picks 32-row groups (one workgroup per CU), 16-row groups, and five pairs per wave."""
    G = 128
    Wq, S = synth.weights(N, K, G, seed=N + M)
    X = synth.activations(M, K, seed=K - M, per_row_seed=True)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("N,K,G", [(64, 96, 32), (130, 320, 64), (48, 768, 256), (32, 1152, 384),
                                   (16, 128, 128), (17, 65536 + 128, 128)])
def test_gemv_shapes_and_groups(kernels, oracle, N, K, G):
    M = 3
    Wq, S = synth.weights(N, K, G, seed=N)
    X = synth.activations(M, K, seed=K)
    y = run_linear(kernels, X, Wq, S, G)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G), 2e-5)


@pytest.mark.parametrize("M,N,K,G", [(128, 128, 128, 128), (256, 384, 1024, 128),
                                     (384, 256, 544, 32), (128, 640, 2048, 256),
                                     (512, 1024, 1056, 32), (512, 768, 1152, 96)])
def test_gemm_small(kernels, oracle, M, N, K, G):
    """Small GEMMs, including the register-staged fallback plans (K % 64 == 32: K = 544, 1056;
    a group size that is not a power of two: G = 96) on grids large enough for its biggest
    tiles."""
    Wq, S = synth.weights(N, K, G, seed=M + K)
    X = synth.activations(M, K, seed=N)
    y = run_linear(kernels, X, Wq, S, G)
    check_close(oracle, y, oracle.linear_f64(X, Wq, S, G), tight=5e-3)
    check_bf16_faithful(y, oracle.linear_f64(X, Wq, S, G, bf16_weights=True), 2e-5)


def _gemm_full_check(kernels, oracle, M, N, K, G, seed):
    """Prefill GEMM on the GPU. The float64 oracle checks one row in every 64-row band of M (the
    smallest M-tile of any GEMM plan, so every output tile of every plan is sampled), every
    column; every row and column is checked against a plain torch fp32 matmul on the GPU with
    the same bf16-staged weights, bf16_rne((q - 8) s)."""
    Wq, S = synth.weights(N, K, G, seed=seed)
    X = synth.activations(M, K, seed=7)
    y = run_linear(kernels, X, Wq, S, G)
    band = 64
    rows = np.array([b * band + (37 * b + 5) % band for b in range(M // band)])
    ref = oracle.linear_f64(X[rows], Wq, S, G)
    check_close(oracle, y[rows], ref, tight=5e-3)
    check_bf16_faithful(y[rows], oracle.linear_f64(X[rows], Wq, S, G, bf16_weights=True), 2e-5)
    # all rows: torch fp32 reference on the GPU (staged weights rounded by torch's RNE cast)
    wq, s = to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=wq.device)
    q = ((wq.unsqueeze(-1) >> shifts) & 0xF).reshape(N, K).float() - 8.0
    w = (q.view(N, K // G, G) * s.float().unsqueeze(-1)).view(N, K).to(torch.bfloat16).float()
    full = (to_dev(X, torch.bfloat16).float() @ w.t()).cpu().numpy().astype(np.float64)
    del q, w
    check_bf16_faithful(y, full, 3e-5)


@pytest.mark.parametrize("name,N,K", [s for s in synth.QWEN7B_LAYERS if s[0] in ("gate_up", "down")],
                         ids=["gate_up", "down"])
@pytest.mark.parametrize("M", [512, 2048])
def test_gemm_configs_sampled_rows(kernels, oracle, name, N, K, M):
    """Full-size config-4 GEMMs (each M picks a different tile plan: 128 x 128, 256 x 128, the
    64 x 128 and 256 x 128 K splits inside the workgroup)."""
    print(f"gemm full-size {name} M={M}", flush=True)
    _gemm_full_check(kernels, oracle, M, N, K, 128, seed=N + K)


@pytest.mark.parametrize("M,N,K", [(1536, 4224, 8192), (2048, 4096, 14336), (512, 4096, 14336),
                                   (256, 3584, 18944), (256, 3584, 3584), (128, 7168, 3584),
                                   (512, 7936, 1024), (1024, 3584, 18944), (768, 4608, 3584),
                                   (1024, 4096, 14336)])
def test_gemm_ksplit_plans(kernels, oracle, M, N, K):
    """The plans that split K inside the workgroup, on shapes besides the config-4 ones (tile
    counts for MI355X's 256 CUs): 256 x 128 tiles over two wave groups (198 tiles, fewer than the
    CUs, at the shortest K the plan takes; 256 tiles of a Llama-3-8B down projection), 128 x 64
    tiles over four groups (256 tiles), 64 x 64 tiles over four groups (224 tiles at long and
    short K, 224 with N = 7168), and 128 x 128 tiles over two groups of four where those fill more
    than half the CUs (248 tiles at K = 1024, 224 at K = 18944, 216, and exactly one round, 256)."""
    print(f"gemm ksplit M={M} N={N} K={K}", flush=True)
    _gemm_full_check(kernels, oracle, M, N, K, 128, seed=M + N)


# ----------------------------------------------------------------- quantizer
@pytest.mark.parametrize("N,K,G", [(64, 512, 128), (33, 96, 32), (16, 768, 96), (8, 2048, 1024),
                                   (300, 3584, 128)])
def test_quantize_bitexact(kernels, oracle, N, K, G):
    rng = np.random.default_rng(N * K)
    w = rng.standard_normal((N, K)).astype(np.float32) * np.float32(0.05)
    w[0, :G] = 0.0                                            # all-zero group
    w[1, :G] = 0.0
    w[1, 3] = -2.5                                            # single nonzero
    if N > 2:
        w[2, :G] = np.round(np.linspace(-7, 7, G)) * 0.125    # exact .5 ties of w / s
    Wb = oracle.f32_to_bf16(w)
    Wq_ref, S_ref = oracle.quantize(Wb, G)
    Wq, S = kernels.w4_quantize(to_dev(Wb, torch.bfloat16), G)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host_bits(S), S_ref)
    np.testing.assert_array_equal(to_host_bits(Wq), Wq_ref)


# ----------------------------------------------------------------- wrapper semantics
def test_wrapper_pads_like_the_reference(kernels, oracle):
    """M = 130 is padded with zero rows to 256 (reference ops.py:89-91); output keeps M rows."""
    M, N, K, G = 130, 256, 256, 128
    Wq, S = synth.weights(N, K, G, seed=1)
    X = synth.activations(M, K, seed=2)
    y = run_linear(kernels, X, Wq, S, G)
    assert y.shape == (M, N)
    check_close(oracle, y, oracle.linear_f64(X, Wq, S, G), tight=5e-3)


def test_wrapper_raises_on_unsupported(kernels):
    x = torch.zeros(1, 100, dtype=torch.bfloat16, device="cuda")   # K % 32 != 0
    Wq = torch.zeros(16, 12, dtype=torch.int32, device="cuda")
    S = torch.ones(16, 1, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="code -2"):
        kernels.w4_linear(x, Wq, S, 100)


def test_repeat_runs_are_bitwise_deterministic(kernels):
    N, K, G = 4608, 3584, 128
    Wq, S = synth.weights(N, K, G, seed=11)
    X = synth.activations(8, K, seed=12)
    xd, wd, sd = to_dev(X, torch.bfloat16), to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    a = to_host_bits(kernels.w4_linear(xd, wd, sd, G))
    b = to_host_bits(kernels.w4_linear(xd, wd, sd, G))
    np.testing.assert_array_equal(a, b)


# ----------------------------------------------------------------- committed golden fixtures
def _golden(name):
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name + ".npz")
    with np.load(path) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("M", [1, 3, 8])
def test_golden_ref_case_gemv(kernels, M):
    c = _golden("ref_case")
    y = run_linear(kernels, c["X"][:M], c["Wq"], c["S"], int(c["G"]))
    check_bf16_faithful(y, c["y_exact"][:M].astype(np.float64), 1e-5)


def test_golden_edge_case(kernels):
    c = _golden("edge_case")
    G = int(c["G"])
    Wq, S = kernels.w4_quantize(to_dev(c["W"], torch.bfloat16), G)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_host_bits(Wq), c["Wq"])
    np.testing.assert_array_equal(to_host_bits(S), c["S"])
    y = run_linear(kernels, c["X"], c["Wq"], c["S"], G)
    check_bf16_faithful(y, c["y_exact"].astype(np.float64), 1e-5)

"""The C-ABI library loads and exports every entry point include/*.h declares.

Runs without a GPU: only host-side entry points (version, workspace queries,
argument validation that returns before any HIP call) are invoked.
"""
import ctypes
import glob
import os
import re
import shutil
import subprocess

import pytest

from chronicals_amd import _lib
from chronicals_amd import build as _build

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w]*\s*\**\s+\**\s*(cce_\w+)\s*\(", re.M)


def declared_functions():
    names = set()
    for hdr in glob.glob(os.path.join(REPO, "include", "*.h")):
        names.update(DECL.findall(open(hdr).read()))
    return names


def header_define(name):
    for hdr in glob.glob(os.path.join(REPO, "include", "*.h")):
        m = re.search(rf"#define\s+{name}\s+(\d+)", open(hdr).read())
        if m:
            return int(m.group(1))
    raise KeyError(name)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.lib_path()):
        pytest.fail(f"{_lib.lib_path()} is not built: run __graft_entry__.build()")
    return _lib.load()


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ("cce_forward", "cce_backward", "cce_forward_workspace_bytes", "cce_backward_workspace_bytes",
              "cce_last_error", "cce_abi_version"):
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert set(_lib.SIGNATURES) <= declared_functions()


def test_no_undeclared_exports():
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", _lib.lib_path()], capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.split() and ln.split()[-1].startswith("cce_")}
    assert exported == declared_functions()


def test_constants_match_header():
    for name in ("CCE_ABI_VERSION", "CCE_OK", "CCE_ERR_INVALID_ARG", "CCE_ERR_WORKSPACE", "CCE_ERR_HIP",
                 "CCE_REDUCTION_NONE", "CCE_REDUCTION_MEAN", "CCE_REDUCTION_SUM", "CCE_DTYPE_BF16",
                 "CCE_DTYPE_F32", "CCE_DTYPE_F16", "CCE_SMOOTH_LOGV", "CCE_SMOOTH_UNIFORM", "CCE_LSE_ALL_ROWS",
                 "CCE_LSE_LABELLED_ROWS", "CCE_KERNEL_FWD_LSE",
                 "CCE_KERNEL_BWD_GRAD", "CCE_KERNEL_BWD_DH", "CCE_KERNEL_BWD_DW", "CCE_KERNEL_BWD_DHDW",
                 "CCE_KERNEL_BWD_BAND", "CCE_KERNEL_LOGITS_FWD", "CCE_KERNEL_LOGITS_BWD", "CCE_KERNEL_LOGITS_FUSED",
                 "CCE_KERNEL_KINDS"):
        assert getattr(_lib, name) == header_define(name), name
    assert sorted(_lib.KERNEL_KIND_NAMES) == list(range(_lib.CCE_KERNEL_KINDS))


def test_kernel_timing_hook_without_launches(lib):
    # nothing recorded: zero time, launches and FLOPs, no device call
    for k in range(_lib.CCE_KERNEL_KINDS):
        assert _lib.kernel_timing_read(k) == (0.0, 0, 0.0, 0.0)
    with pytest.raises(_lib.CCEError, match="out of range"):
        _lib.kernel_timing_read(_lib.CCE_KERNEL_KINDS)
    import ctypes
    ms, n = ctypes.c_double(), ctypes.c_int64()
    # the FLOP outputs are optional
    assert lib.cce_kernel_timing_read(0, ctypes.byref(ms), ctypes.byref(n), None, None) == _lib.CCE_OK
    assert lib.cce_kernel_timing_read(0, None, ctypes.byref(n), None, None) == _lib.CCE_ERR_INVALID_ARG


def test_abi_version(lib):
    assert lib.cce_abi_version() == header_define("CCE_ABI_VERSION")


def test_library_built_from_the_tree(lib):
    """The build compiles the SHA-256 of its sources into the library, and
    the loaded in-tree library carries the tree's."""
    h = lib.cce_source_hash().decode()
    assert re.fullmatch(r"[0-9a-f]{64}", h), h
    assert h == _build.source_hash()


def test_source_hash_follows_the_sources(tmp_path):
    # any edit of the kernel file or the header changes the hash
    src = tmp_path / "cce_kernels.hip"
    src.write_bytes(open(_build.SRC, "rb").read() + b"// edit\n")
    hdr = tmp_path / "chronicals_cce.h"
    hdr.write_bytes(open(_build.HEADER, "rb").read().replace(b"CCE_OK 0", b"CCE_OK  0"))
    base = _build.source_hash()
    assert _build.source_hash((str(src), _build.HEADER)) != base
    assert _build.source_hash((_build.SRC, str(hdr))) != base
    assert _build.source_hash((_build.SRC, _build.HEADER)) == base


def test_stale_library_is_refused(lib, monkeypatch):
    # a tree whose sources changed after the build: the loader refuses the
    # in-tree library, and accepts it again once the hashes agree
    monkeypatch.setattr(_build, "source_hash", lambda *a, **k: "0" * 64)
    with pytest.raises(ImportError, match="built from other sources"):
        _lib.check_fresh(lib, _build.LIB_PATH)
    # a library named explicitly (CHRONICALS_CCE_LIB) is the caller's choice
    _lib.check_fresh(lib, "/elsewhere/libchronicals_cce.so")
    monkeypatch.undo()
    _lib.check_fresh(lib, _build.LIB_PATH)


@pytest.mark.parametrize("d,V", [(896, 151936), (4096, 128256), (768, 50257), (3584, 152064)])
def test_small_batch_backward_workspace_bounded(lib, d, V):
    """Small batches widen the vocabulary bands (from 1024 rows) and split dH
    into fp32 partials (few row tiles); neither may make a smaller batch need
    more backward workspace than 4096 rows at the same chunk_size, and below
    1024 rows none of it may outgrow the materialised fp32 logits and their
    gradient."""
    ref = _lib.backward_workspace_bytes(4096, d, V, 8192, True, True)
    for N in (1, 256, 512, 1024, 2048, 3072):
        ws = _lib.backward_workspace_bytes(N, d, V, 8192, True, True)
        assert 0 < ws <= ref, (N, ws, ref)
    if d <= 1024:
        assert _lib.backward_workspace_bytes(256, d, V, 8192, True, True) < 256 * V * 8


def test_workspace_queries(lib):
    f1 = _lib.forward_workspace_bytes(1024, 896, 151936, _lib.CCE_REDUCTION_MEAN)
    f2 = _lib.forward_workspace_bytes(2048, 896, 151936, _lib.CCE_REDUCTION_MEAN)
    assert 0 < f1 < f2
    # forward scratch is O(N): the row partials, never N x V
    assert f2 < 2048 * 151936
    b = _lib.backward_workspace_bytes(16384, 896, 151936, 8192, True, True)
    # at least one band of G (N x chunk bf16), far below N x V
    assert 16384 * 8192 * 2 <= b < 16384 * 151936 * 2
    b_frozen = _lib.backward_workspace_bytes(16384, 896, 151936, 8192, True, False)
    assert b_frozen < b
    # empty batch is a valid problem
    assert _lib.forward_workspace_bytes(0, 64, 300, _lib.CCE_REDUCTION_MEAN) > 0
    assert _lib.forward_workspace_bytes(0, 64, 300, _lib.CCE_REDUCTION_NONE) > 0
    assert _lib.backward_workspace_bytes(0, 64, 300, 8192, True, True) >= 0
    # chunk_size bounds the band from above; the band is at most 8192 columns
    # (the trainer's get_optimal_chunk_size gives 16384 at V >= 128K)
    assert _lib.backward_workspace_bytes(16384, 896, 151936, 2048, True, True) < b
    assert _lib.backward_workspace_bytes(16384, 896, 151936, 16384, True, True) == b
    assert (_lib.backward_workspace_bytes(64, 64, 2 ** 22, 2 ** 22, True, True)
            == _lib.backward_workspace_bytes(64, 64, 2 ** 22, 2 ** 20, True, True))
    assert _lib.forward_workspace_bytes(2 ** 21, 64, 1000, _lib.CCE_REDUCTION_MEAN) > 0  # the largest N
    # fp32 gradients accumulate in place: no fp32 dH / dW accumulators
    assert _lib.backward_workspace_bytes(16384, 896, 151936, 8192, True, True, True, True) < b


def test_compacted_forward_partials_bounded(lib, monkeypatch):
    """A labelled-rows forward launches room for up to 64 vocabulary splits
    per row tile for the device to choose from, but no more than 8192
    workgroups beyond the all-rows count: each workgroup holds a 256-row slot
    of (max, sum-exp) partials (2 KiB), so at the largest N the partials stay
    near 16 MiB instead of 64 splits x N x 8 B = 1 GiB.  Counted here with
    the row copy forced off (rows read in place), the rest being O(N) row
    data."""
    monkeypatch.setenv("CHRONICALS_CCE_ROW_GATHER", "1")
    V = 151936
    for N, d in ((2 ** 21 // 4, 256), (2 ** 20, 128)):
        lab = _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS)
        every = _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_ALL_ROWS)
        assert lab - every <= 8192 * 256 * 8 + N * 4 + 4096, (N, d, lab, every)
    # at the benchmark sizes the device keeps its full choice: 64 slots per
    # row tile at C2 (64 row tiles), 8192 workgroups at C5 (256 row tiles)
    for N, d, V, slots in ((16384, 896, 151936, 64 * 64), (65536, 3584, 152064, 8192)):
        lab = _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS)
        every = _lib.forward_workspace_bytes(N, d, V, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_ALL_ROWS)
        s_all = max(-(-512 // (N // 256)), min(32, -(-2048 // (N // 256))))
        assert lab - every >= (slots - s_all * (N // 256)) * 256 * 8, (N, lab, every)


@pytest.mark.parametrize("d,V", [(896, 151936), (3584, 152064), (128, 50257)])
def test_backward_band_gradient_bounded_in_N(lib, d, V):
    """The band gradient G (two bf16 buffers of rows x band) is processed in
    row blocks within a 512 MiB budget, so past one block the workspace grows
    only by the O(N*d) buffers (the fp32 dH accumulator and, past 2 GiB of H,
    H in row order: at most 8*d bytes per row; H's transpose lives in
    grad_hidden until dH is written) and the O(N) row data, never by
    N*band."""
    per_row = 8 * d + 64
    n1, n2 = 2 ** 17, 2 ** 21
    w1 = _lib.backward_workspace_bytes(n1, d, V, 8192, True, True)
    w2 = _lib.backward_workspace_bytes(n2, d, V, 8192, True, True)
    # at both batches, all but the O(N*d) buffers fit in the G budget plus
    # the band's W^T (two buffers), its fp32 dW accumulator and the fp32
    # partials of a K-split dH (about 128 tiles of 256 x 256, two buffers)
    band_rest = 512 * 2 ** 20 + 2 * d * 8192 * 2 + 8192 * d * 4 + 2 * 160 * 256 * 256 * 4 + 2 ** 20
    assert w1 - n1 * per_row <= band_rest
    assert w2 - n2 * per_row <= band_rest
    assert w2 - w1 >= (n2 - n1) * 4 * d  # the O(N*d) buffers are there
    # a query for a gradient dtype other than bf16 / fp32 is refused
    out = ctypes.c_size_t(0)
    assert lib.cce_backward_workspace_bytes(1024, d, V, 8192, 1, 7, 1, 0, ctypes.byref(out)) == \
        _lib.CCE_ERR_INVALID_ARG


def test_backward_workspace_borrows_gradient_memory(lib):
    """While the bands run, grad_hidden holds H^T (bf16 dH, several bands) or,
    with no dW wanted, the two band transposes of W; the rows of band b+1 of
    grad_weight hold band b's W^T.  None of it takes workspace: C5 needs
    under 1.5 GiB, the transposes no longer count at C2, and fp32 dH (the
    output is its own accumulator) keeps H^T in the workspace."""
    c2 = (16384, 896, 151936)
    c5 = (65536, 3584, 152064)
    w5 = _lib.backward_workspace_bytes(*c5, 8192, True, True)
    assert w5 <= 1536 * 2 ** 20, w5 / 2 ** 20
    N, d, V = c5
    # G (two 16384-row blocks of one 8192-column band), the fp32 dH
    # accumulator, the fp32 dW band accumulator and the O(N) row data
    assert w5 <= 2 * 16384 * 8192 * 2 + N * d * 4 + 8192 * d * 4 + N * 64 + 2 ** 20
    w2 = _lib.backward_workspace_bytes(*c2, 8192, True, True)
    N, d, V = c2
    # one band of W^T (the last band's) besides G, the dH accumulator, H in
    # row order (a copy below 256 MiB) and the row data
    assert w2 <= 2 * N * 8192 * 2 + N * d * 4 + d * 8192 * 2 + N * d * 2 + N * 64 + 2 ** 20
    assert _lib.backward_workspace_bytes(*c2, 8192, True, False) < w2  # frozen W
    w2_f32 = _lib.backward_workspace_bytes(*c2, 8192, True, True, True, False)
    assert w2_f32 >= w2 - N * d * 4 + d * N * 2  # no dH accumulator, but H^T in the workspace


def test_row_order_copy_policy(lib, monkeypatch):
    """The compacted GEMMs read H through the row order when H takes 256 MiB
    to 2 GiB (the byte offsets fit 32 bits and a gathered copy would be
    large); below that, above it, or with CHRONICALS_CCE_ROW_GATHER=0 both
    workspaces hold a gathered N x d bf16 copy of H.  =1 reads in place
    wherever the offsets fit."""
    def both(N, d):
        return (_lib.backward_workspace_bytes(N, d, 152064, 8192, True, True),
                _lib.forward_workspace_bytes(N, d, 152064, _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_LABELLED_ROWS))
    cases = {"C2": (16384, 896), "C5": (65536, 3584), "large": (2 ** 21, 1024)}   # H: 28 MiB, 448 MiB, 4 GiB
    ws = {}
    for env in (None, "0", "1"):
        if env is None:
            monkeypatch.delenv("CHRONICALS_CCE_ROW_GATHER", raising=False)
        else:
            monkeypatch.setenv("CHRONICALS_CCE_ROW_GATHER", env)
        for k, nd in cases.items():
            ws[k, env] = both(*nd)
    def copy(k):
        return cases[k][0] * cases[k][1] * 2
    for i in range(2):
        assert ws["C5", "0"][i] - ws["C5", None][i] == copy("C5")   # C5: in place by default
        assert ws["C5", "1"][i] == ws["C5", None][i]
        assert ws["C2", None][i] - ws["C2", "1"][i] == copy("C2")   # C2: the copy by default
        assert ws["C2", "0"][i] == ws["C2", None][i]
        assert ws["large", "1"][i] == ws["large", "0"][i] == ws["large", None][i]   # past 2 GiB: always the copy


@pytest.mark.parametrize("N,d,V,red,msg", [
    (16, 7, 100, 1, "multiple of 8"),
    (16, 0, 100, 1, "multiple of 8"),
    (16, 64, 0, 1, "vocab"),
    (-1, 64, 10, 1, "N must be"),
    (16, 64, 100, 5, "reduction"),
    (2 ** 21 + 1, 64, 100, 1, "too large"),   # tokens per call
    (16, 2 ** 20 + 8, 100, 1, "too large"),
    (16, 64, 2 ** 30 + 1, 1, "too large"),
])
def test_workspace_query_rejects_bad_arguments(lib, N, d, V, red, msg):
    out = ctypes.c_size_t(0)
    rc = lib.cce_forward_workspace_bytes(N, d, V, red, _lib.CCE_LSE_ALL_ROWS, ctypes.byref(out))
    assert rc == _lib.CCE_ERR_INVALID_ARG
    assert msg in lib.cce_last_error().decode()


def test_lse_rows_option(lib):
    out = ctypes.c_size_t(0)
    assert lib.cce_forward_workspace_bytes(64, 64, 1000, 1, 2, ctypes.byref(out)) == _lib.CCE_ERR_INVALID_ARG
    assert "lse_rows" in lib.cce_last_error().decode()
    fake = 0x10000
    rc = lib.cce_forward(fake, fake, fake, 1, None, 64, 64, 1000, -100, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV,
                         _lib.CCE_REDUCTION_MEAN, 7, fake, fake, None, fake, fake, 1 << 30, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "lse_rows" in lib.cce_last_error().decode()
    # labelled rows only: with d a multiple of 64 the forward reorders the rows (the row order in the
    # workspace; the GEMM reads H through it); with any other d it needs nothing more
    sizes = {}
    for d in (64, 72):
        for rows in (_lib.CCE_LSE_ALL_ROWS, _lib.CCE_LSE_LABELLED_ROWS):
            assert lib.cce_forward_workspace_bytes(300, d, 1000, 1, rows, ctypes.byref(out)) == _lib.CCE_OK
            sizes[d, rows] = out.value
    assert sizes[64, 1] >= sizes[64, 0] + 300 * 4
    assert sizes[72, 1] == sizes[72, 0]


def test_forward_rejects_small_workspace_before_launch(lib):
    fake = 0x10000  # never dereferenced: validation fails first
    rc = lib.cce_forward(fake, fake, fake, 1, None, 64, 64, 1000, -100, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV,
                         _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_ALL_ROWS, fake, fake, None, fake, fake, 16, None)
    assert rc == _lib.CCE_ERR_WORKSPACE
    assert "workspace too small" in lib.cce_last_error().decode()


def test_forward_rejects_null_inputs(lib):
    rc = lib.cce_forward(None, None, None, 1, None, 64, 64, 1000, -100, 0.0, 0.0, _lib.CCE_SMOOTH_LOGV,
                         _lib.CCE_REDUCTION_MEAN, _lib.CCE_LSE_ALL_ROWS, 0x10000, 0x10000, None, 0x10000, 0x10000,
                         1 << 20, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG


def test_forward_rejects_bad_smoothing_form(lib):
    fake = 0x10000
    rc = lib.cce_forward(fake, fake, fake, 1, None, 64, 64, 1000, -100, 0.1, 0.0, 2, _lib.CCE_REDUCTION_MEAN,
                         _lib.CCE_LSE_ALL_ROWS, fake, fake, None, fake, fake, 1 << 30, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "smoothing_form" in lib.cce_last_error().decode()
    rc = lib.cce_logits_forward(fake, 0, 1000, fake, 1, 64, 1000, -100, 0.1, 0.0, 5, 1, fake, fake, fake, fake,
                                1 << 30, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "smoothing_form" in lib.cce_last_error().decode()


def test_backward_rejects_bad_dtype_and_bias(lib):
    fake = 0x10000
    rc = lib.cce_backward(fake, fake, fake, fake, 1, None, fake, fake, 64, 64, 1000, -100, 0.0, 0.0, 1, 8192,
                          fake, 7, None, 0, None, fake, 1 << 30, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "dtype" in lib.cce_last_error().decode()
    rc = lib.cce_backward(fake, fake, fake, fake, 1, None, fake, fake, 64, 64, 1000, -100, 0.0, 0.0, 1, 8192,
                          fake, 0, None, 0, fake, fake, 1 << 30, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "bias" in lib.cce_last_error().decode()


def test_misaligned_pointers_rejected(lib):
    rc = lib.cce_forward(0x10002, 0x10000, 0x10000, 1, None, 64, 64, 1000, -100, 0.0, 0.0, 0, 1, 0,
                         0x10000, 0x10000, None, 0x10000, 0x10000, 1 << 20, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "aligned" in lib.cce_last_error().decode()


def test_build_command_targets_gfx950():
    cmd = _build.compile_command("/tmp/x.so")
    assert "--offload-arch=gfx950" in cmd
    assert "-packed-fp32-ops" in cmd


def test_built_kernels_do_not_spill():
    """The build records each kernel's compiler resource report: no kernel may spill VGPRs to
    scratch (a spill reload inside the pipeline would also wait on the outstanding slab DMA), and
    every kernel fits the 160 KB of LDS a workgroup can have."""
    from chronicals_amd import build as _build
    if not os.path.exists(_build.RESOURCES_PATH):
        pytest.skip("library not built in this tree")
    kernels = {}
    with open(_build.RESOURCES_PATH) as f:
        for line in f:
            name, *fields = line.split()
            kernels[name] = dict(kv.split("=", 1) for kv in fields)
    assert any("band_kernel" in n for n in kernels) and any("gemm_kernel" in n for n in kernels)
    for name, r in kernels.items():
        assert int(r.get("VGPRs_Spill", 0)) == 0, f"{name} spills {r['VGPRs_Spill']} VGPRs"
        assert int(r.get("LDS_Size_[bytes/block]", 0)) <= 160 * 1024, name


def test_missing_library_fails_loudly(tmp_path):
    # no fallback: without the built HIP library the package raises instead of computing elsewhere
    import subprocess
    import sys
    code = ("from chronicals_amd import _lib\n"
            "try:\n    _lib.load()\nexcept ImportError as e:\n    print('IMPORT_ERROR', e)\n")
    env = dict(os.environ, CHRONICALS_CCE_LIB=str(tmp_path / "absent.so"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, cwd=REPO,
                         timeout=300)
    assert "IMPORT_ERROR" in out.stdout and "not found" in out.stdout, out.stdout + out.stderr


def test_gradient_may_alias_logits_only_with_same_layout(lib):
    fake = 0x10000
    # fp32 gradient written over bf16 logits: refused before any launch
    rc = lib.cce_logits_backward(fake, fake, _lib.CCE_DTYPE_BF16, 1000, fake, 1, fake, fake, 64, 1000, -100, 0.0, 0.0,
                                 _lib.CCE_SMOOTH_LOGV, 1, fake, _lib.CCE_DTYPE_F32, 1000, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "alias" in lib.cce_last_error().decode()
    rc = lib.cce_logits_forward_backward(fake, _lib.CCE_DTYPE_BF16, 1000, fake, 1, 64, 1000, -100, 0.0, 0.0,
                                         _lib.CCE_SMOOTH_LOGV, 1, 1, fake, fake, fake, fake, _lib.CCE_DTYPE_BF16, 1024,
                                         fake, 1 << 20, None)
    assert rc == _lib.CCE_ERR_INVALID_ARG and "alias" in lib.cce_last_error().decode()


def test_plain_c_caller_compiles_links_and_queries(tmp_path):
    """The boundary is plain C: a C99 program that includes the header
    compiles with -pedantic, links against the library and makes a workspace
    query (no device work), which matches the Python binding's."""
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "caller.c"
    src.write_text(
        "#include \"chronicals_cce.h\"\n#include <stdio.h>\n"
        "int main(void) {\n  size_t b = 0;\n"
        "  int rc = cce_forward_workspace_bytes(16384, 896, 151936, CCE_REDUCTION_MEAN, CCE_LSE_LABELLED_ROWS, &b);\n"
        "  printf(\"%d %zu %d\\n\", rc, b, cce_abi_version());\n  return rc;\n}\n")
    libdir = os.path.dirname(_build.LIB_PATH)
    exe = tmp_path / "caller"
    cmd = [gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.join(REPO, "include"), str(src),
           "-L", libdir, "-lchronicals_cce", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert int(out[0]) == _lib.CCE_OK
    assert int(out[1]) == _lib.forward_workspace_bytes(16384, 896, 151936, _lib.CCE_REDUCTION_MEAN,
                                                        _lib.CCE_LSE_LABELLED_ROWS)
    assert int(out[2]) == _lib.CCE_ABI_VERSION

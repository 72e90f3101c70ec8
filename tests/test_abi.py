"""The C ABI (include/rk_path.h) without a GPU: the library loads, exports every declared function, the ctypes
signatures agree with the header's parameter lists, and argument errors come back as status codes with a message
(validation happens before any HIP call, so these run on any machine)."""
import ctypes
import re
from pathlib import Path

import pytest

from native import rocm_native
from native.rocm_native import SIGNATURES, NativeRocm

HEADER = Path(__file__).resolve().parents[1] / "include" / "rk_path.h"
PROBE_HEADER = HEADER.with_name("rk_probe.h")


def declarations(header: Path = HEADER) -> dict[str, list[str]]:
    """name -> list of parameter declarations, for every function prototype in the header."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^[\w\s\*]*?\b(rk_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        params = [p.strip() for p in m.group(2).replace("\n", " ").split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = params
    return out


def kind(param: str) -> str:
    if "*" in param:
        return "char*" if param.startswith("char") else "ptr"
    t = param.rsplit(" ", 1)[0]
    return {"int": "int", "size_t": "size_t", "float": "float", "long long": "long long"}[t]


CTYPE_KIND = {ctypes.c_void_p: "ptr", ctypes.c_char_p: "char*", ctypes.c_int: "int", ctypes.c_size_t: "size_t",
              ctypes.c_float: "float", ctypes.c_longlong: "long long"}


@pytest.fixture(scope="module")
def lib():
    if not rocm_native.LIB_PATH.exists():
        pytest.fail(f"{rocm_native.LIB_PATH} is not built (run __graft_entry__.build())")
    return NativeRocm()


def test_header_and_binding_declare_the_same_functions():
    assert set(declarations()) == set(SIGNATURES)


@pytest.mark.parametrize("name", sorted(SIGNATURES))
def test_signature_matches_header(name):
    params = declarations()[name]
    _, argtypes = SIGNATURES[name]
    assert [kind(p) for p in params] == [CTYPE_KIND[a] for a in argtypes], name


def test_every_declared_symbol_is_exported(lib):
    for name in declarations():
        assert hasattr(lib.lib, name), name
    assert lib.lib.rk_abi_version() == rocm_native.ABI_VERSION


def test_probe_library_matches_its_header():
    decl = declarations(PROBE_HEADER)
    assert set(decl) == set(rocm_native.PROBE_SIGNATURES)
    for name, (_, argtypes) in rocm_native.PROBE_SIGNATURES.items():
        assert [kind(p) for p in decl[name]] == [CTYPE_KIND[a] for a in argtypes], name
    probes = rocm_native.load_probes()
    for name in decl:
        assert hasattr(probes.lib, name), name
    rc = probes.lib.rk_probe_block_stream(None, None, None, 0, 16384, 1, 0, None, None)
    assert rc == 1 and b"rk_probe_block_stream" in probes.lib.rk_last_error()


def test_null_pointer_is_an_argument_error(lib):
    rc = lib.lib.rk_paged_decode(None, None, None, None, 1, None, None, 1, 8, 2, 256, 16, 1, 1, 0, None, 0, None, 0,
                                 None)
    assert rc == 1 and "null pointer" in lib.last_error()


def test_unsupported_shapes_are_refused(lib):
    fake = 4096                            # never dereferenced: validation fails first
    rc = lib.lib.rk_paged_decode(fake, fake, fake, fake, 1, fake, fake, 1, 8, 2, 96, 16, 1, 1, 0, None, 0, fake,
                                 1 << 20, None)
    assert rc == 2 and "head_dim 96" in lib.last_error()
    rc = lib.lib.rk_paged_decode(fake, fake, fake, fake, 7, fake, fake, 1, 8, 2, 256, 16, 1, 1, 0, None, 0, fake,
                                 1 << 20, None)
    assert rc == 2 and "dtype" in lib.last_error()
    rc = lib.lib.rk_paged_decode(fake, fake, fake, fake, 1, fake, fake, 1, 9, 2, 256, 16, 1, 1, 0, None, 0, fake,
                                 1 << 20, None)
    assert rc == 1
    rc = lib.lib.rk_paged_decode(fake, fake, fake, fake, 1, fake, fake, 1, 8, 2, 256, 16, 1, 1, 0, fake, 8 * 256 - 4,
                                 fake, 1 << 20, None)
    assert rc == 1 and "gate rows" in lib.last_error()
    rc = lib.lib.rk_paged_decode(fake, fake, fake, fake, 1, fake, fake, 1, 8, 2, 256, 16, 1, 1, 0, fake, 8 * 256 + 2,
                                 fake, 1 << 20, None)
    assert rc == 1 and "gate rows" in lib.last_error()
    args = [fake] * 5 + [6144, 2048, 16] + [fake] * 7 + [8, 16, 64, 64, 4, 1, 0, ctypes.c_float(1e-6), None]
    assert lib.lib.rk_deltanet_decode(*args) == 2 and "dk 64" in lib.last_error()
    args = [fake] * 5 + [6144, 2048, 16] + [fake] * 7 + [8, 16, 128, 128, 4, 2, 2, ctypes.c_float(1e-6), None]
    assert lib.lib.rk_deltanet_decode(*args) == 1 and "slot 2" in lib.last_error()
    args = [fake] * 5 + [6143, 2048, 16] + [fake] * 7 + [8, 16, 128, 128, 4, 2, 0, ctypes.c_float(1e-6), None]
    assert lib.lib.rk_deltanet_decode(*args) == 1 and "row strides" in lib.last_error()


def test_too_small_workspace_is_refused(lib):
    fake = 4096
    rc = lib.lib.rk_paged_decode(fake, fake, fake, fake, 1, fake, fake, 64, 8, 2, 256, 16, 512, 20000, 0, None, 0,
                                 fake, 16, None)
    assert rc == 3 and "workspace" in lib.last_error()


def test_gather_table_bounds_checked_on_host(lib):
    fake = 4096
    rc = lib.lib.rk_kv_gather(fake, fake, fake, fake, 1, fake, 2, 0, 40, 2, 64, 16, 8, None)
    assert rc == 1 and "table" in lib.last_error()


def test_empty_work_is_a_no_op(lib):
    assert lib.lib.rk_kv_write(None, None, 1, None, None, None, 0, 0, 2, 64, 16, 8, None) == 0
    assert lib.lib.rk_kv_gather(None, None, None, None, 1, None, 0, 5, 5, 2, 64, 16, 8, None) == 0


def test_workspace_size_formula(lib):
    """(waves + B * Hkv) partial records of GP * (D + 2) floats; waves = min(units upper bound, 8 per CU)."""
    n = lib.lib.rk_paged_decode_workspace_bytes(64, 8, 2, 256, 16, 512)
    assert n > 0 and n % (4 * (256 + 2) * 4) == 0
    assert lib.lib.rk_paged_decode_workspace_bytes(0, 8, 2, 256, 16, 512) == 0


def test_paged_prefill_checked_on_host(lib):
    """rk_paged_prefill refuses bad shapes and short workspaces before any launch: head_dim 96 (no instance), query
    heads that do not split over the kv-heads, position counts past 2^31, and split partials / counters below the
    size functions' figures. Any group size and head_dim 64 / 128 / 256 pass validation (reached here only with an
    invalid dtype, refused next)."""
    fake = 4096

    def call(Hq=8, Hkv=2, D=256, max_nb=4, bs=16, q_dtype=0, n_slots=0, part_bytes=0, n_cnt=0, exact=0):
        return lib.lib.rk_paged_prefill(fake, fake, q_dtype, fake, fake, 0, fake, fake, 0, fake, max_nb, fake, fake,
                                        fake, 1, 1, 8, Hq, Hkv, D, bs, 64, None, 0, 0, 1, exact, n_slots,
                                        fake if n_slots else None, part_bytes, fake if n_slots else None, n_cnt, None)
    assert call(D=96) == 2 and "head_dim 96" in lib.last_error()
    assert call(Hq=6, Hkv=4) == 1 and "6 query heads" in lib.last_error()
    assert call(max_nb=1 << 20, bs=4096) == 2 and "2^31" in lib.last_error()
    for Hq, Hkv, D in ((14, 2, 64), (8, 8, 128), (32, 4, 256), (7, 1, 64)):
        assert call(Hq, Hkv, D, q_dtype=7) == 2 and "dtype 7" in lib.last_error()
    need = lib.lib.rk_paged_prefill_workspace_bytes(3, 8, 256)
    cnt = lib.lib.rk_paged_prefill_counters(3, 8)
    assert need == 3 * 8 * (32 * 256 + 64) * 4 and cnt == 3 * 8 * 2
    assert call(n_slots=3, part_bytes=need - 4, n_cnt=cnt) == 3 and "partial bytes" in lib.last_error()
    assert call(n_slots=3, part_bytes=need, n_cnt=cnt - 1) == 3
    assert call(n_slots=3, part_bytes=need, n_cnt=cnt, q_dtype=7) == 2            # sizes accepted, dtype refused
    assert lib.lib.rk_paged_prefill_workspace_bytes(0, 8, 256) == 0 and lib.lib.rk_paged_prefill_counters(0, 8) == 0


def test_gated_delta_arguments_checked_on_host(lib):
    fake = 4096
    ws = lib.lib.rk_gated_delta_workspace_bytes(256, 16)
    assert ws == 256 * 16 * (2 * 3 * 3072 * 2 + 4 * 64 * 4) and lib.lib.rk_gated_delta_workspace_bytes(-1, 16) == 0

    def call(**kw):
        a = dict(out=fake, S=fake, stride=16 * 128 * 128, q=fake, k=fake, v=fake, dt=1, beta=fake, g=fake, cu=fake,
                 cuc=fake, idx=None, n=4, chunks=256, H=16, dk=128, dv=128, ws=fake, wsb=ws)
        a.update(kw)
        return lib.lib.rk_gated_delta_chunked(*a.values(), None)

    assert call(q=None) == 1 and "null pointer" in lib.last_error()
    assert call(dk=64) == 2 and "dk 64" in lib.last_error()
    assert call(dt=7) == 2 and "dtype" in lib.last_error()
    assert call(stride=128) == 1 and "stride" in lib.last_error()
    assert call(wsb=ws - 1) == 3 and "workspace" in lib.last_error()


def test_deltanet_prefill_companions_checked_on_host(lib):
    fake = 4096
    C = 6144

    def front(**kw):
        a = dict(q=fake, k=fake, v=fake, beta=fake, g=fake, qkv=fake, b=fake, a=fake, dt=1, ld=C + 2048 + 32,
                 conv=fake, cs=3 * C, w=fake, A=fake, dtb=fake, cu=fake, idx=fake, n=4, N=100, H=16, dk=128, dv=128,
                 K=4)
        a.update(kw)
        return lib.lib.rk_deltanet_prefill_front(*a.values(), None)

    assert front(qkv=None) == 1 and "null pointer" in lib.last_error()
    assert front(conv=None) == 1 and "null pointer" in lib.last_error()
    assert front(dk=64) == 2 and "dk 64" in lib.last_error()
    assert front(dt=5) == 2 and "dtype 5" in lib.last_error()
    assert front(K=9) == 1 and "conv kernel 9" in lib.last_error()
    assert front(ld=C - 2) == 1 and "row stride" in lib.last_error()
    assert front(cs=3 * C - 2) == 1 and "state stride" in lib.last_error()
    assert front(ld=C + 1) == 1 and "aligned" in lib.last_error()
    assert front(qkv=fake + 2, dt=0) == 1 and "aligned" in lib.last_error()
    assert front(N=0) == 0                                           # nothing to do
    assert lib.lib.rk_causal_conv1d(fake, fake, fake, 0, C, fake, fake, 5, C, 1, None) == 1
    assert "K 1" in lib.last_error()
    assert lib.lib.rk_causal_conv1d(fake, fake, fake, 0, C - 1, fake, fake, 5, C, 4, None) == 1
    assert lib.lib.rk_causal_conv1d(fake, fake, fake, 3, C, fake, fake, 5, C, 4, None) == 2
    assert lib.lib.rk_rms_norm_gated(fake, fake, fake, 0, 128, 1, fake, 10, 96, 1e-6, None) == 1
    assert "dv 96" in lib.last_error()
    assert lib.lib.rk_rms_norm_gated(fake, fake, fake, 0, 16 * 128 - 1, 16, fake, 32, 128, 1e-6, None) == 1
    assert lib.lib.rk_rms_norm_gated(fake, fake, fake, 2, 128, 1, fake, 10, 128, 1e-6, None) == 2
    assert lib.lib.rk_rms_norm_gated(None, None, None, 0, 128, 1, None, 0, 128, 1e-6, None) == 0


def test_attn_prep_checked_on_host(lib):
    fake = 4096

    def call(**kw):
        a = dict(q=fake, k=None, v=None, kp=fake, vp=fake, pdt=1, slots=fake, nb=256, bs=16, y=fake, ydt=0,
                 ld=12 * 256 + 8 * 256, qw=fake, kw=fake, eps=1e-6, pos=fake, inv=fake, rot=64, N=64, Hq=8, Hkv=2,
                 d=256)
        a.update(kw)
        return lib.lib.rk_attn_prep(*a.values(), None)

    assert call(q=None) == 1 and "null pointer" in lib.last_error()
    assert call(kp=None) == 1 and "null pointer" in lib.last_error()
    assert call(inv=None) == 1 and "null pointer" in lib.last_error()
    assert call(d=96) == 2 and "head_dim 96" in lib.last_error()
    assert call(rot=48) == 2 and "rotary dims 48" in lib.last_error()
    assert call(rot=512) == 2
    assert call(ld=11 * 256) == 1 and "row stride" in lib.last_error()
    assert call(ydt=3) == 2 and "dtypes" in lib.last_error()
    assert call(pdt=4) == 2
    assert call(y=fake + 4) == 1 and "aligned" in lib.last_error()
    assert call(N=0) == 0


def test_linear_arguments_checked_on_host(lib):
    fake = 4096

    def call(**kw):
        a = dict(y=fake, x=fake, M=8, N=2048, K=2048, w=fake, wt=2, s=fake, m=fake, b=None, r=None, p=fake,
                 pb=1 << 30, c=fake, nc=128)
        a.update(kw)
        return lib.lib.rk_linear_rows(*a.values(), None)

    assert call(wt=7) == 2 and "weight type 7" in lib.last_error()
    assert call(M=17) == 1 and "M 17" in lib.last_error()
    assert call(K=2047) == 1
    assert call(wt=3, m=None) == 1 and "null pointer" in lib.last_error()
    assert call(y=fake + 4, x=fake + 8) == 1 and "aligned" in lib.last_error()
    # (K = 4096: quantized K = 2048 at up to 8 rows runs whole-K workgroups with no workspace, and would launch)
    need = lib.lib.rk_linear_workspace_bytes(8, 2048, 4096, 2)
    assert need == 4 * 8 * 2048 * 4                            # 4 K-splits of 32 blocks
    assert call(K=4096, pb=need - 1) == 3 and "partials" in lib.last_error()
    assert call(K=4096, nc=127) == 3 and "counters" in lib.last_error()    # 128 groups of 16 rows
    assert lib.lib.rk_linear_workspace_bytes(8, 2048, 1024, 2) == 0      # one split: no workspace
    assert lib.lib.rk_linear_workspace_bytes(12, 2048, 2048, 1) == 2 * 12 * 2048 * 4
    assert lib.lib.rk_linear_workspace_bytes(3, 100, 6144, 3) == 6 * 3 * 100 * 4
    assert lib.lib.rk_linear_workspace_bytes(12, 2048, 2048, 3) == 2 * 12 * 2048 * 4
    assert call(M=0) == 0
    assert lib.lib.rk_dequant_rows(fake, fake, 2, fake, None, None, 10, 5, 12, 2048, None) == 1
    assert "rows 10 + 5 of 12" in lib.last_error()


def test_decode_ops_checked_on_host(lib):
    fake = 4096
    L = lib.lib
    for fn in (L.rk_rms_norm, L.rk_layer_norm):
        assert fn(fake, None, 0, 2048, fake, 0, 4, 2048, 1e-6, None) == 1                      # null x
        assert fn(fake, fake, 5, 2048, fake, 0, 4, 2048, 1e-6, None) == 2                      # x dtype
        assert fn(fake, fake, 0, 2048, fake, 0, 4, 0, 1e-6, None) == 1                         # D < 1
        assert fn(fake, fake, 0, 1024, fake, 0, 4, 2048, 1e-6, None) == 1                      # stride < D
        assert "row stride" in lib.last_error()
        assert fn(fake, fake, 0, 2048, fake, 0, -1, 2048, 1e-6, None) == 1                     # negative rows
        assert fn(fake, fake, 0, 2048, fake, 0, 0, 2048, 1e-6, None) == 0                      # no rows
    assert L.rk_rope(fake, fake, fake, fake, 3, 2, 63, None) == 1 and "even" in lib.last_error()
    assert L.rk_rope(fake, fake, None, fake, 3, 2, 64, None) == 1
    assert L.rk_rope(fake, fake, fake, fake, 0, 2, 64, None) == 0
    assert L.rk_silu_mul(fake, fake, 100, fake, 200, 4, 128, None) == 1 and "strides" in lib.last_error()
    assert L.rk_silu_mul(fake, None, 256, fake, 256, 4, 128, None) == 1
    assert L.rk_silu_mul(fake, fake, 256, fake, 256, 0, 128, None) == 0


def test_linear_ex_checked_on_host(lib):
    fake = 4096
    L = lib.lib

    def call(**kw):
        a = dict(y=fake, x=fake, xld=4096, op=1, aux=fake + 8192, auxld=4096, M=8, N=2048, K=2048, w=fake, wt=3,
                 s=fake, m=fake, b=None, r=None, p=fake, pb=1 << 30, c=fake, nc=1024)
        a.update(kw)
        return L.rk_linear_rows_ex(*a.values(), None)

    assert call(op=3) == 1 and "input transform 3" in lib.last_error()
    assert call(aux=None) == 1 and "null pointer" in lib.last_error()
    assert call(M=9) == 2 and "M <= 8" in lib.last_error()
    assert call(K=2080, xld=4160, auxld=4160) == 2                  # K % 256 != 0
    assert call(xld=2047) == 1 and "stride" in lib.last_error()
    assert call(auxld=100) == 1 and "up rows" in lib.last_error()
    assert call(M=0) == 0


def test_linear_ex2_checked_on_host(lib):
    """rk_linear_rows_ex2's RMSNorm transform: the norm weight, the K and row limits and the sums' stride are checked
    before any launch; rk_linear_rows_ex does not take the transform."""
    fake = 4096
    L = lib.lib

    def call(**kw):
        a = dict(y=fake, ss=None, x=fake, xld=2048, op=2, aux=fake + 8192, auxld=128, nw=fake, eps=1e-6, M=8, N=2048,
                 K=2048, w=fake, wt=3, s=fake, m=fake, b=None, r=None, p=fake, pb=1 << 30, c=fake, nc=1024)
        a.update(kw)
        return L.rk_linear_rows_ex2(*a.values(), None)

    assert call(nw=None) == 1 and "norm weight" in lib.last_error()
    assert call(nw=fake + 4) == 1 and "norm weight" in lib.last_error()
    assert call(auxld=127) == 1 and "sums of squares" in lib.last_error()
    assert call(K=4096, xld=4096, auxld=256) == 1 and "sums of squares" in lib.last_error()
    assert call(M=9) == 2 and "M <= 8" in lib.last_error()
    sw = dict(y=fake, x=fake, xld=2048, op=2, aux=fake + 8192, auxld=128, nw=fake, eps=1e-6, M=8, F=6144, K=2048,
              w=fake, wt=3, s=fake, m=fake, p=fake, pb=1 << 30, c=fake, nc=1024)

    def swiglu(**kw):
        return L.rk_swiglu_rows(*dict(sw, **kw).values(), None)

    assert swiglu(op=1) == 1 and "input transform 1" in lib.last_error()
    assert swiglu(F=6148) == 2 and "multiple of 8" in lib.last_error()
    assert swiglu(nw=None) == 1 and "norm weight" in lib.last_error()
    assert swiglu(M=9) == 2 and "M <= 8" in lib.last_error()
    assert swiglu(M=0) == 0 and swiglu(F=0) == 0
    ex = dict(y=fake, x=fake, xld=2048, op=2, aux=fake, auxld=2048, M=8, N=2048, K=2048, w=fake, wt=3, s=fake, m=fake,
              b=None, r=None, p=fake, pb=1 << 30, c=fake, nc=1024)
    assert L.rk_linear_rows_ex(*ex.values(), None) == 1 and "input transform 2" in lib.last_error()

"""The C ABI (CPU only: no kernel is launched).

The library loads without a GPU, exports every function include/ declares,
and rejects invalid descriptors, null pointers and short workspaces on the
host with the documented status codes and a message, before any launch.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

import femtochat_amd._lib as L

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "femtochat_attn.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions(header=None):
    names = set()
    for h in ([header] if header else HEADERS):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(fc_[a-z_0-9]+)\s*\(", text))
    return sorted(names)


def test_exports_every_declared_symbol():
    lib = L.lib()
    names = declared_functions()
    assert len(names) >= 15, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
        assert n in L._SIGNATURES, f"{n} has no ctypes signature"


def test_header_compiles_as_c_and_cpp():
    assert len(HEADERS) >= 2
    for h in HEADERS:
        for lang, cc in (("c", "gcc"), ("c++", "g++")):
            r = subprocess.run([cc, "-x", lang, "-fsyntax-only", "-Wall", "-Werror", str(h)], capture_output=True,
                               text=True)
            assert r.returncode == 0, (h.name, r.stderr)


def test_abi_version_and_head_dims():
    lib = L.lib()
    assert lib.fc_abi_version() == 1
    mask = lib.fc_attn_supported_head_dims()
    dims = [16 * (i + 1) for i in range(8) if (mask >> i) & 1]
    # every multiple of 16 up to 128, as the reference's tensor-core path takes (ext/FemtoChatCUDAExt.jl:214-223)
    assert dims == [16, 32, 48, 64, 80, 96, 112, 128]


@pytest.mark.parametrize("D,Dk", [(48, 64), (80, 128), (96, 128), (112, 128)])
@pytest.mark.parametrize("mode", [L.FC_MODE_FAST, L.FC_MODE_EXACT])
def test_padded_head_dims_need_their_copies_in_the_workspace(D, Dk, mode):
    """Head dims between the compiled widths run on zero-padded copies: the
    forward's workspace grows by Q, K, V and O of width Dk (and becomes
    required), the backward's by those plus dO and float32 dQ, dK, dV; a
    compiled width asks for none of it."""
    t = L.FC_BF16 if mode == L.FC_MODE_FAST else L.FC_F32
    B, T, H, Hkv = 2, 64, 4, 2
    e = 2 if t == L.FC_BF16 else 4
    nq, nk = B * T * H * Dk, B * T * Hkv * Dk

    def a256(x):
        return (x + 255) // 256 * 256

    kw = dict(D=D, H=H, Hkv=Hkv, T=T, B=B, mode=mode, in_dtype=t, out_dtype=t, dout_dtype=t, grad_dtype=t)
    st, fwd = ws_bytes(desc(**kw), L.FC_PASS_FORWARD)
    assert st == L.FC_OK
    assert fwd == a256(nq * e) + 2 * a256(nk * e) + a256(nq * e)
    st, bwd = ws_bytes(desc(**kw))
    st_c, bwd_c = ws_bytes(desc(**dict(kw, D=Dk)))
    assert st == st_c == L.FC_OK
    pads = a256(nq * e) * 3 + 2 * a256(nk * e) + a256(nq * 4) + 2 * a256(nk * 4)
    assert bwd == pads + bwd_c
    assert ws_bytes(desc(**dict(kw, D=Dk)), L.FC_PASS_FORWARD)[1] == 0
    # the forward of a padded head dim refuses to run without its workspace (checked before any launch)
    fake = ctypes.c_void_p(0x1000)
    st = L.lib().fc_attn_fwd(ctypes.byref(desc(**kw)), fake, fake, fake, None, fake, fake, fake, None, 0, None)
    assert st == L.FC_ERR_WORKSPACE and "padded" in L.lib().fc_last_error().decode()


def desc(**kw):
    d = L.AttnDesc()
    base = dict(D=128, H=4, Hkv=2, T=64, B=2, win_left=-1, win_right=0, mode=L.FC_MODE_FAST,
                in_dtype=L.FC_BF16, out_dtype=L.FC_BF16, dout_dtype=L.FC_BF16, grad_dtype=L.FC_BF16, flags=0)
    base.update(kw)
    for k, v in base.items():
        setattr(d, k, v)
    return d


def ws_bytes(d, pass_=L.FC_PASS_BACKWARD, pos=0):
    n = ctypes.c_size_t(0)
    st = L.lib().fc_attn_workspace_bytes(ctypes.byref(d), pass_, pos, ctypes.byref(n))
    return st, n.value


BAD = [
    (dict(H=5, Hkv=2), L.FC_ERR_INVALID_ARGUMENT, "multiple"),
    (dict(D=24), L.FC_ERR_INVALID_ARGUMENT, "head_dim"),
    (dict(D=256), L.FC_ERR_INVALID_ARGUMENT, "head_dim"),
    (dict(T=0), L.FC_ERR_INVALID_ARGUMENT, "positive"),
    (dict(B=-1), L.FC_ERR_INVALID_ARGUMENT, "positive"),
    (dict(mode=7), L.FC_ERR_INVALID_ARGUMENT, "mode"),
    (dict(in_dtype=L.FC_F32), L.FC_ERR_INVALID_ARGUMENT, "bfloat16"),
    (dict(mode=L.FC_MODE_EXACT), L.FC_ERR_INVALID_ARGUMENT, "float32"),
    (dict(out_dtype=9), L.FC_ERR_INVALID_ARGUMENT, "dtype"),
    (dict(flags=0x10), L.FC_ERR_INVALID_ARGUMENT, "flag"),
]


@pytest.mark.parametrize("kw,status,msg", BAD, ids=[str(b[0]) for b in BAD])
def test_invalid_descriptors(kw, status, msg):
    st, _ = ws_bytes(desc(**kw))
    assert st == status
    assert msg in L.lib().fc_last_error().decode()
    fake = ctypes.c_void_p(0x1000)
    st = L.lib().fc_attn_fwd(ctypes.byref(desc(**kw)), fake, fake, fake, None, fake, fake, fake, None, 0, None)
    assert st == status


def test_null_descriptor_and_pointers():
    lib = L.lib()
    n = ctypes.c_size_t(0)
    assert lib.fc_attn_workspace_bytes(None, 0, 0, ctypes.byref(n)) == L.FC_ERR_INVALID_ARGUMENT
    fake = ctypes.c_void_p(0x1000)
    d = desc()
    assert lib.fc_attn_fwd(ctypes.byref(d), None, fake, fake, None, fake, fake, fake, None, 0, None) == \
        L.FC_ERR_INVALID_ARGUMENT
    assert "null" in lib.fc_last_error().decode()
    st = lib.fc_attn_bwd(ctypes.byref(d), fake, fake, fake, fake, fake, fake, fake, None, None, fake, fake, fake,
                         0, None)
    assert st == L.FC_ERR_INVALID_ARGUMENT


def test_convert_rejects_overlapping_buffers():
    """fc_convert runs restrict-qualified kernels: any overlap other than an
    in-place copy of one dtype is rejected on the host (no launch)."""
    lib = L.lib()
    base = 0x100000
    n = 1024
    # in place with different dtypes: thread i would write bytes thread i/2 still reads
    for sd, dd in ((L.FC_F32, L.FC_BF16), (L.FC_BF16, L.FC_F32)):
        st = lib.fc_convert(ctypes.c_void_p(base), sd, ctypes.c_void_p(base), dd, ctypes.c_int64(n), None)
        assert st == L.FC_ERR_INVALID_ARGUMENT
        assert "overlap" in lib.fc_last_error().decode()
    # partial overlap, equal dtypes
    st = lib.fc_convert(ctypes.c_void_p(base), L.FC_F32, ctypes.c_void_p(base + 64), L.FC_F32, ctypes.c_int64(n), None)
    assert st == L.FC_ERR_INVALID_ARGUMENT
    # a bf16 destination just below an fp32 source of the same count, one byte into it
    st = lib.fc_convert(ctypes.c_void_p(base + 2 * n - 2), L.FC_F32, ctypes.c_void_p(base), L.FC_BF16,
                        ctypes.c_int64(n), None)
    assert st == L.FC_ERR_INVALID_ARGUMENT


def test_workspace_checks():
    lib = L.lib()
    d = desc()
    st, need = ws_bytes(d)
    assert st == L.FC_OK and need > 0
    st, fwd = ws_bytes(d, L.FC_PASS_FORWARD)
    assert st == L.FC_OK and fwd == 0
    # delta + lse2 (fp32 per query) at least; positions add the chunk bounds.
    assert need >= 2 * 4 * d.B * d.H * d.T
    _, need_pos = ws_bytes(d, pos=1)
    assert need_pos > need
    # fp32 dO in fast mode adds a bf16 copy of dO.
    _, need_f32 = ws_bytes(desc(dout_dtype=L.FC_F32))
    assert need_f32 >= need + 2 * d.B * d.T * d.H * d.D
    fake = ctypes.c_void_p(0x1000)
    st = lib.fc_attn_bwd(ctypes.byref(d), fake, fake, fake, fake, fake, fake, fake, None, fake, fake, fake, fake,
                         need - 1, None)
    assert st == L.FC_ERR_WORKSPACE
    assert str(need) in lib.fc_last_error().decode()
    st = lib.fc_attn_bwd(ctypes.byref(d), fake, fake, fake, fake, fake, fake, fake, None, fake, fake, fake,
                         ctypes.c_void_p(0x1001), need, None)
    assert st == L.FC_ERR_WORKSPACE and "aligned" in lib.fc_last_error().decode()


def test_forward_workspace_for_the_work_order():
    """Only fast mode with positions has a forward workspace (chunk bounds and
    the query-tile order), and only while the order tables fit (B * ceil(T/128)
    <= 4096); the backward then holds the dQ and dK/dV orders as well."""
    lib = L.lib()

    def fwd_bytes(d, pos):
        st, n = ws_bytes(d, L.FC_PASS_FORWARD, pos=pos)
        assert st == L.FC_OK
        return n

    d = desc(T=1000, B=3)
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    chunk = align(3 * 32 * 2 * 4)  # ceil(1000/32) = 32 chunks of (min, max)
    order = align(3 * 8 * 4)       # ceil(1000/128) = 8 tiles per row
    assert fwd_bytes(d, 0) == 0
    assert fwd_bytes(d, 1) == chunk + order
    exact = desc(T=1000, B=3, mode=L.FC_MODE_EXACT, in_dtype=L.FC_F32, out_dtype=L.FC_F32, dout_dtype=L.FC_F32,
                 grad_dtype=L.FC_F32)
    assert fwd_bytes(exact, 1) == 0
    assert fwd_bytes(desc(T=64 * 8192, B=1, H=1, Hkv=1, D=16), 1) > 0
    assert fwd_bytes(desc(T=64 * 8192 + 1, B=1, H=1, Hkv=1, D=16), 1) == 0
    _, bwd_pos = ws_bytes(d, pos=1)
    _, bwd_exact = ws_bytes(exact, pos=1)
    assert bwd_pos >= 2 * 4 * 3 * 4 * 1000 + chunk + 2 * order
    # A workspace is optional for the forward, but a short or misaligned one is an error.
    fake = ctypes.c_void_p(0x1000)
    need = fwd_bytes(d, 1)
    st = lib.fc_attn_fwd(ctypes.byref(d), fake, fake, fake, fake, fake, fake, fake, fake, need - 1, None)
    assert st == L.FC_ERR_WORKSPACE and str(need) in lib.fc_last_error().decode()
    st = lib.fc_attn_fwd(ctypes.byref(d), fake, fake, fake, fake, fake, fake, fake, ctypes.c_void_p(0x1001), need,
                         None)
    assert st == L.FC_ERR_WORKSPACE and "aligned" in lib.fc_last_error().decode()
    # Exact mode: Delta, lse2 and the chunk bounds, no work counters or orders.
    assert bwd_exact == 2 * align(4 * 3 * 4 * 1000) + chunk


def test_noalloc_backward_rejects_problems_beyond_its_scratch():
    # Checked on the host before any HIP call: B*H*T = 2^23 query rows need
    # 2 * 4 * 2^23 bytes = 64 MiB of statistics, above the 32 MiB scratch.
    lib = L.lib()
    fake = ctypes.c_void_p(0x1000)
    big = desc(D=16, H=128, Hkv=128, T=65536, B=1)
    st, need = ws_bytes(big)
    assert st == L.FC_OK and need > 32 << 20
    st = lib.fc_attn_bwd_noalloc(ctypes.byref(big), fake, fake, fake, fake, fake, fake, fake, None, fake, fake,
                                 fake, None)
    assert st == L.FC_ERR_WORKSPACE
    msg = lib.fc_last_error().decode()
    assert str(need) in msg and str(32 << 20) in msg
    st = lib.fc_attn_bwd_noalloc(ctypes.byref(desc()), fake, fake, fake, fake, fake, fake, fake, None, None, fake,
                                 fake, None)
    assert st == L.FC_ERR_INVALID_ARGUMENT and "fc_attn_bwd_noalloc" in lib.fc_last_error().decode()


def test_last_error_is_cleared_on_success():
    lib = L.lib()
    ws_bytes(desc(H=5, Hkv=2))
    assert lib.fc_last_error().decode() != ""
    st, _ = ws_bytes(desc())
    assert st == L.FC_OK and lib.fc_last_error().decode() == ""


def test_profile_collect_empty():
    L.profile_enable(False)
    assert L.profile_collect() == {}


def _xent(**kw):
    d = L.XentDesc()
    d.V, d.N, d.index_base, d.ignore_index = kw.get("V", 100), kw.get("N", 8), kw.get("index_base", 0), -1
    d.index_type, d.reduction, d.flags = kw.get("index_type", 0), kw.get("reduction", 2), kw.get("flags", 0)
    return d


@pytest.mark.parametrize("kw,msg", [
    (dict(V=0), "positive"), (dict(N=0), "positive"), (dict(index_base=2), "index_base"),
    (dict(index_type=3), "index_type"), (dict(reduction=5), "reduction"), (dict(flags=4), "flag"),
])
def test_cross_entropy_rejects_bad_descriptors(kw, msg):
    lib = L.lib()
    fake = ctypes.c_void_p(0x1000)
    st = lib.fc_cross_entropy_fwd(ctypes.byref(_xent(**kw)), fake, fake, fake, None, None, None, None)
    assert st == L.FC_ERR_INVALID_ARGUMENT
    assert msg in lib.fc_last_error().decode()


def test_cross_entropy_pointer_checks():
    lib = L.lib()
    fake = ctypes.c_void_p(0x1000)
    d = _xent()
    assert lib.fc_cross_entropy_fwd(ctypes.byref(d), fake, None, fake, None, None, None, None) == L.FC_ERR_INVALID_ARGUMENT
    assert lib.fc_cross_entropy_fwd(ctypes.byref(d), None, fake, fake, None, None, None, None) == L.FC_ERR_INVALID_ARGUMENT
    # the mean gradient needs the valid-target count
    assert lib.fc_cross_entropy_bwd(ctypes.byref(d), fake, fake, fake, fake, None, None, None) == L.FC_ERR_INVALID_ARGUMENT
    assert "count" in lib.fc_last_error().decode()
    # misaligned int64 targets
    d64 = _xent(index_type=1)
    assert lib.fc_cross_entropy_fwd(ctypes.byref(d64), fake, ctypes.c_void_p(0x1004), fake, None, None, None,
                                    None) == L.FC_ERR_INVALID_ARGUMENT
    assert lib.fc_cross_entropy_count(ctypes.byref(d), fake, None, None) == L.FC_ERR_INVALID_ARGUMENT


def test_embedding_rejects_bad_descriptors():
    lib = L.lib()
    fake = ctypes.c_void_p(0x1000)
    d = L.EmbedDesc()
    d.D, d.vocab, d.N, d.index_base, d.index_type, d.y_dtype, d.flags = 64, 100, 8, 0, 0, 0, 0
    for field, bad in (("D", 0), ("vocab", -1), ("N", 0), ("index_base", 3), ("y_dtype", 7), ("flags", 1)):
        e = L.EmbedDesc.from_buffer_copy(d)
        setattr(e, field, bad)
        assert lib.fc_embedding_fwd(ctypes.byref(e), fake, fake, fake, None) == L.FC_ERR_INVALID_ARGUMENT, field
        assert lib.fc_embedding_bwd(ctypes.byref(e), fake, fake, fake, None) == L.FC_ERR_INVALID_ARGUMENT, field
    assert lib.fc_embedding_fwd(ctypes.byref(d), None, fake, fake, None) == L.FC_ERR_INVALID_ARGUMENT
    assert lib.fc_embedding_bwd(ctypes.byref(d), fake, None, fake, None) == L.FC_ERR_INVALID_ARGUMENT


def test_fast_mode_rejects_slices_past_32_bit_offsets():
    # The fast kernels address one (batch, head) slice with 32-bit buffer
    # offsets: (T-1)*H*D*2 + 2*D bytes must stay below 2^31.
    lib = L.lib()
    D, H = 128, 10
    t_max = ((1 << 31) - 2 * D - 1) // (H * D * 2) + 1  # largest T whose slice fits
    st, _ = ws_bytes(desc(D=D, H=H, Hkv=5, T=t_max, B=1))
    assert st == L.FC_OK, lib.fc_last_error().decode()
    st, _ = ws_bytes(desc(D=D, H=H, Hkv=5, T=t_max + 1, B=1))
    assert st == L.FC_ERR_UNSUPPORTED and "2^31" in lib.fc_last_error().decode()
    fake = ctypes.c_void_p(0x1000)
    d = desc(D=D, H=H, Hkv=5, T=t_max + 1, B=1)
    assert lib.fc_attn_fwd(ctypes.byref(d), fake, fake, fake, None, fake, fake, fake, None, 0, None) == \
        L.FC_ERR_UNSUPPORTED
    # exact mode addresses with 64-bit offsets and has no such bound
    st, _ = ws_bytes(desc(D=D, H=H, Hkv=5, T=t_max + 1, B=1, mode=L.FC_MODE_EXACT, in_dtype=L.FC_F32,
                          out_dtype=L.FC_F32, dout_dtype=L.FC_F32, grad_dtype=L.FC_F32))
    assert st == L.FC_OK


def test_grouped_polar_express_checks_every_stack_before_launching():
    # The second stack's workspace is too small: the call fails on the host
    # with FC_ERR_WORKSPACE before the first stack is enqueued (no GPU needed).
    lib = L.lib()
    descs = (L.PolarDesc * 2)()
    for d in descs:
        d.m, d.n, d.count, d.steps, d.dtype = 64, 32, 2, 5, L.FC_F32
    need = ctypes.c_size_t(0)
    assert lib.fc_polar_workspace_bytes(ctypes.byref(descs[0]), ctypes.byref(need)) == L.FC_OK
    fake = ctypes.c_void_p(0x100000)
    G = (ctypes.c_void_p * 2)(fake, fake)
    ws = (ctypes.c_void_p * 2)(fake, fake)
    nbytes = (ctypes.c_size_t * 2)(need.value, need.value - 1)
    st = lib.fc_polar_express_grouped(2, descs, G, ws, nbytes, None)
    assert st == L.FC_ERR_WORKSPACE and str(need.value) in lib.fc_last_error().decode()
    nbytes = (ctypes.c_size_t * 2)(need.value, need.value)
    ws = (ctypes.c_void_p * 2)(fake, ctypes.c_void_p(0x100040))
    st = lib.fc_polar_express_grouped(2, descs, G, ws, nbytes, None)
    assert st == L.FC_ERR_WORKSPACE and "aligned" in lib.fc_last_error().decode()

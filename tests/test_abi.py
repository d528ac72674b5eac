"""C-ABI library: loads without a GPU, exports every symbol the header declares,
and its host-only planner satisfies the work-list invariants (CPU only)."""
import ctypes
import re

import numpy as np
import pytest

from conftest import ROOT
from oracle import plan as oplan

HEADER = ROOT / "include" / "mi355x_attn.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi355x_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def native():
    from llm_infer_rust_amd import _native
    return _native


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("mi355x_store_kv", "mi355x_rms_norm", "mi355x_add_rms_norm",
                     "mi355x_qk_norm", "mi355x_decode_prepare", "mi355x_decode_run",
                     "mi355x_decode_plan_drop", "mi355x_prefill_prepare", "mi355x_prefill_run",
                     "mi355x_prefill_plan_drop"):
        assert required in names


def test_library_exports_every_declared_symbol(native):
    lib = native.lib()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared but not exported"
    assert set(native.SIGNATURES) == set(declared_functions())
    assert lib.mi355x_attn_abi_version() == 1


def _schedule(native, lengths, cus=256, hkv=8):
    lib = native.lib()
    lens = (ctypes.c_int32 * len(lengths))(*lengths)
    cap = lib.mi355x_decode_items_capacity(len(lengths), cus, hkv)
    work = (ctypes.c_int32 * (4 * cap))()
    merge = (ctypes.c_int32 * (2 * len(lengths)))()
    chunk = ctypes.c_int64()
    n = lib.mi355x_decode_schedule(lens, len(lengths), cus, hkv, work, cap, merge,
                                   ctypes.byref(chunk))
    return n, list(work)[: 4 * max(n, 0)], list(merge), chunk.value, cap


@pytest.mark.parametrize("seed", range(6))
def test_decode_schedule_invariants(native, seed):
    rng = np.random.default_rng(seed)
    b = int(rng.choice([1, 3, 64, 256, 700]))
    lengths = rng.integers(1, 8192, size=b).tolist()
    n, work, merge, chunk, cap = _schedule(native, lengths)
    assert 0 < n <= cap
    oplan.check_work_list(work, merge, lengths)
    assert chunk % 16 == 0 or chunk == max(lengths)


def test_decode_schedule_config2_shape(native):
    rng = np.random.default_rng(2)
    lengths = rng.integers(512, 4097, size=64).tolist()
    n, work, merge, chunk, cap = _schedule(native, lengths)
    oplan.check_work_list(work, merge, lengths)
    # at least one item per CU, each share a bounded slice of the KV
    assert n >= 256
    assert chunk >= 128


def test_decode_schedule_cuts_on_tiles(native):
    """Shares are counted in the decode kernels' 16-token tiles plus a per-item cost: cuts
    fall on tile boundaries, and a batch of nearly equal requests (the config-5 decode
    shape) is not cut at all."""
    rng = np.random.default_rng(2)
    lengths = rng.integers(512, 4097, size=64).tolist()
    n, work, merge, chunk, cap = _schedule(native, lengths)
    items = np.array(work).reshape(-1, 4)
    assert (items[:, 1] % 16 == 0).all()
    assert n <= 256 + len(lengths)  # one cut per share boundary at most
    lengths = (1280 + rng.integers(-32, 33, size=256)).tolist()
    n, work, merge, chunk, cap = _schedule(native, lengths)
    oplan.check_work_list(work, merge, lengths)
    assert n == 256 and all(c == 1 for c in merge[1::2])


def test_decode_schedule_randomized_batches(native):
    """The tile-counted share search and the whole-request placement over a wide spread of
    batches: a few very long requests, many one-token requests, mixtures, up to 2,048 rows."""
    rng = np.random.default_rng(31)
    for case in range(120):
        b = int(rng.choice([1, 2, 5, 17, 64, 200, 256, 257, 700, 2048]))
        kind = case % 4
        if kind == 0:
            lengths = rng.integers(1, 17, size=b)
        elif kind == 1:
            lengths = rng.integers(1, 1 << 20, size=b) if b <= 17 else rng.integers(1, 9000, size=b)
        elif kind == 2:
            lengths = 1280 + rng.integers(-40, 41, size=b)
        else:
            lengths = np.where(rng.random(b) < 0.1, rng.integers(4000, 70000, size=b),
                               rng.integers(1, 300, size=b))
        lengths = lengths.astype(int).tolist()
        n, work, merge, chunk, cap = _schedule(native, lengths)
        assert 0 < n <= cap, (case, b, kind)
        oplan.check_work_list(work, merge, lengths)


def test_decode_schedule_rejects_bad_input(native):
    lib = native.lib()
    lens = (ctypes.c_int32 * 2)(5, 0)
    work = (ctypes.c_int32 * 64)()
    merge = (ctypes.c_int32 * 4)()
    chunk = ctypes.c_int64()
    assert lib.mi355x_decode_schedule(lens, 2, 256, 8, work, 16, merge, ctypes.byref(chunk)) == -1
    lens = (ctypes.c_int32 * 1)(10**6)
    assert lib.mi355x_decode_schedule(lens, 1, 256, 8, work, 1, merge, ctypes.byref(chunk)) == -1


def test_linear_workspace_bytes_query(native):
    f = native.lib().mi355x_linear_workspace_bytes
    assert f(256, 4096, 4096, 256, 6, 1) == 0
    assert f(256, 4096, 4096, 256, 6, 4) == 4 * 256 * 4096 * 4
    assert f(0, 4096, 4096, 256, -1, -1) == -1
    # the library's own choice for the Qwen3-8B down projection splits K
    assert f(256, 4096, 12288, 256, -1, -1) > 0


@pytest.mark.parametrize("ragged", [False, True])
@pytest.mark.parametrize("seed", range(5))
def test_prefill_schedule_covers_every_query_block_once(native, seed, ragged):
    """mi355x_prefill_schedule: every (request, 32 x waves / heads-per-block query block, kv
    head, head group) appears exactly once, and items come longest causal horizon first.
    Batches with a cached prefix run 8-wave workgroups, batches without one 4-wave ones."""
    rng = np.random.default_rng(seed)
    b = int(rng.integers(1, 12))
    hq, hkv = [(16, 8), (32, 8), (8, 8), (64, 8), (8, 1)][seed]
    q_lens = rng.integers(1, 900, size=b)
    prefixes = rng.integers(0, 3000, size=b) * (rng.random(b) < 0.5) * (not ragged)
    q_host = (ctypes.c_int32 * (b + 1))(*([0] + np.cumsum(q_lens).tolist()))
    p_host = (ctypes.c_int32 * b)(*prefixes.tolist())
    lib = native.lib()
    n = lib.mi355x_prefill_schedule(q_host, p_host, b, hq, hkv, None, 0)
    work = (ctypes.c_int32 * (4 * n))()
    assert lib.mi355x_prefill_schedule(q_host, p_host, b, hq, hkv, work, n) == n
    items = np.array(list(work), dtype=np.int64).reshape(n, 4)
    group = hq // hkv
    waves = 8 if (prefixes > 0).any() else 4
    hpb = min(group, waves)
    bq = 32 * (waves // hpb)
    want = {(r, q0, h, g) for r in range(b) for q0 in range(0, int(q_lens[r]), bq)
            for h in range(hkv) for g in range(group // hpb)}
    got = [tuple(int(v) for v in row) for row in items]
    assert len(got) == len(set(got)) and set(got) == want
    horizon = [int(prefixes[r]) + min(q0 + bq, int(q_lens[r])) for r, q0, _, _ in got]
    tiles = [(h + 63) // 64 for h in horizon]
    assert tiles == sorted(tiles, reverse=True)
    # a capacity below the item count is refused
    assert lib.mi355x_prefill_schedule(q_host, p_host, b, hq, hkv, work, n - 1) == -1


def test_entry_points_reject_bad_arguments_before_launching(native):
    """Argument validation of the compute entries runs on the host and returns the error
    string without touching the device (fake addresses are never dereferenced)."""
    lib = native.lib()
    a, b, c = 0x10000, 0x20000, 0x30000  # 16-byte aligned, never dereferenced

    def err(r):
        assert r is not None
        return r.decode()

    assert "null pointer" in err(lib.mi355x_rms_norm(None, None, None, 4, 1, 128, 128, 128,
                                                      1e-6, 0, None))
    assert "null pointer" in err(lib.mi355x_add_rms_norm(None, b, c, 4, 128, 128, 128, 1e-6,
                                                          0, None))
    assert "alias" in err(lib.mi355x_add_rms_norm(a, a, c, 4, 128, 128, 128, 1e-6, 0, None))
    assert "null pointer" in err(lib.mi355x_qk_norm(a, None, b, c, 4, 2, 1, 128, 384, 128,
                                                     384, 128, 1e-6, 0, None))
    assert "bad shape" in err(lib.mi355x_rms_norm(a, b, c, -1, 1, 128, 128, 128, 1e-6, 0, None))
    # zero tokens is a no-op, not an error
    assert lib.mi355x_rms_norm(None, None, None, 0, 1, 128, 128, 128, 1e-6, 0, None) is None
    assert "null pointer" in err(lib.mi355x_store_kv(a, b, None, c, a, 4, 8, 128, 100, 1024,
                                                      128, 1024, 128, 0, False, None, None))
    assert "invalid geometry" in err(lib.mi355x_store_kv(a, b, c, c, a, 4, 0, 128, 100, 1024,
                                                          128, 1024, 128, 0, False, None, None))
    # projections: K not a multiple of 64, too many rows, split-K without a workspace
    assert "unsupported shape" in err(lib.mi355x_linear(a, 96, b, 96, c, 64, 8, 64, 96, None,
                                                         0, 256, -1, -1, 0, None))
    assert "unsupported shape" in err(lib.mi355x_linear(a, 128, b, 128, c, 64, 4097, 64, 128,
                                                         None, 0, 256, -1, -1, 0, None))
    assert "workspace" in err(lib.mi355x_linear(a, 1024, b, 1024, c, 256, 64, 256, 1024, None,
                                                0, 256, 6, 4, 0, None))
    assert "invalid tile" in err(lib.mi355x_linear(a, 1024, b, 1024, c, 256, 64, 256, 1024,
                                                   None, 0, 256, 99, 1, 0, None))
    # fused projection + residual norm: residual rows narrower than N, out aliasing residual
    assert "width" in err(lib.mi355x_linear_add_rms_norm(a, 4096, b, 4096, c, 2048, a, 1e-6, b,
                                                         4096, 8, 4096, 4096, None, 0, 256, 0,
                                                         None))
    assert "alias" in err(lib.mi355x_linear_add_rms_norm(a, 4096, b, 4096, c, 4096, a, 1e-6, c,
                                                         4096, 8, 4096, 4096, None, 0, 256, 0,
                                                         None))
    assert "null pointer" in err(lib.mi355x_sample(None, 2, 100, 100, 0, None, None, None, 1, 0,
                                                   None, None))
    assert "bad shape" in err(lib.mi355x_silu_mul(a, b, -1, 64, 0, None))


# C parameter / return type (after removing names) -> the Rust FFI type that matches it.
C_TO_RUST = {
    "void*": "*mut c_void", "const void*": "*const c_void", "int64_t": "i64", "int32_t": "i32",
    "int": "c_int", "bool": "bool", "double": "f64", "uint64_t": "u64", "void": "()",
    "const char*": "*const c_char", "int32_t*": "*mut i32", "const int32_t*": "*const i32",
    "int64_t*": "*mut i64", "const int64_t*": "*const i64", "const float*": "*const f32",
}


def header_signatures():
    """name -> (return type, [parameter types]) of every declaration in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, params in re.findall(
            r"([A-Za-z_][\w ]*?\**)\s*\b(mi355x_\w+)\s*\(([^)]*)\)\s*;", text):
        types = []
        for p in [p.strip() for p in params.split(",") if p.strip() and p.strip() != "void"]:
            p = re.sub(r"\s+", " ", p)
            m = re.match(r"(.*?)(\**)\s*\b\w+$", p)
            types.append((m.group(1).strip() + m.group(2)).replace(" *", "*"))
        out[name] = (re.sub(r"\s+", " ", ret.strip()).replace(" *", "*"), types)
    return out


def crate_signatures():
    """name -> (return type, [parameter types]) of the mi355x_sys crate's extern block."""
    text = (ROOT / "rust" / "mi355x_sys" / "src" / "lib.rs").read_text()
    out = {}
    for name, params, ret in re.findall(r"pub fn (mi355x_\w+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;",
                                        text):
        types = [re.sub(r"\s+", " ", p.split(":", 1)[1].strip())
                 for p in params.split(",") if p.strip()]
        out[name] = ((ret or "()").strip(), types)
    return out


def test_rust_crate_declares_every_entry_with_matching_types():
    """The FFI crate a maintainer adds to the reference (rust/mi355x_sys) declares exactly the
    entries of the C header, each parameter and return type the Rust equivalent of the C one."""
    header, crate = header_signatures(), crate_signatures()
    assert set(header) == set(declared_functions())
    assert set(crate) == set(header)
    for name, (ret, params) in header.items():
        cret, cparams = crate[name]
        assert C_TO_RUST[ret] == cret, (name, ret, cret)
        assert [C_TO_RUST[p] for p in params] == cparams, (name, params, cparams)


def test_rust_backend_uses_only_declared_entries():
    """The drop-in backend module calls only entries the crate declares."""
    text = (ROOT / "rust" / "attention_mi355x.rs").read_text()
    used = set(re.findall(r"sys::(mi355x_\w+)\(", text))
    assert used and used <= set(crate_signatures())
    for needed in ("mi355x_decode_prepare", "mi355x_decode_run", "mi355x_decode_plan_drop",
                   "mi355x_prefill_prepare", "mi355x_prefill_run", "mi355x_prefill_plan_drop"):
        assert needed in used

"""Host-side behaviour that needs no GPU: the input contract and its messages,
backend honesty, the storage helpers, the workload byte model, and the C-ABI
library's exported surface."""

import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from flash_decode_int4 import int4_pack, ops, workloads
from flash_decode_int4._validate import normalize_attention_inputs

from conftest import ROOT


def _paged_problem(batch=2, heads=3, dim=32, n_blocks=3, rows=64, seed=0):
    rng = np.random.RandomState(seed)
    query = (rng.randn(batch, heads, dim) / np.sqrt(dim)).astype(np.float32)
    k_q, k_s, k_z, vals = [], [], [], []
    for _ in range(n_blocks):
        k = rng.randn(rows, dim).astype(np.float32)
        v = rng.randn(rows, dim).astype(np.float32)
        q, s_, z = oracle.quantize_int4_ref(k)
        k_q.append(q); k_s.append(s_); k_z.append(z); vals.append(v)
    return query, k_q, k_s, k_z, vals


class TestAttentionInputContract:
    """reference tests/test_ops_dispatch.py:181-243: the same ValueError messages,
    raised before any device work (so they hold on a host without a GPU)."""

    def test_block_len_longer_than_page_is_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem(rows=64)
        with pytest.raises(ValueError, match="outside"):
            ops.flash_decode(query, k_q, k_s, k_z, vals, np.array([64, 65, 64]), backend="hip")

    def test_negative_block_len_is_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem()
        with pytest.raises(ValueError, match="outside"):
            ops.flash_decode(query, k_q, k_s, k_z, vals, np.array([64, -1, 64]), backend="hip")

    def test_wrong_number_of_block_lens_is_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem()
        with pytest.raises(ValueError, match="entries"):
            ops.flash_decode(query, k_q, k_s, k_z, vals, np.array([64, 64]), backend="hip")

    def test_mismatched_page_lists_are_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem()
        with pytest.raises(ValueError, match="same length"):
            ops.flash_decode(query, k_q, k_s, k_z, vals[:-1], backend="hip")

    def test_value_page_shape_mismatch_is_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem()
        vals[1] = vals[1][:-3]
        with pytest.raises(ValueError, match="value page 1"):
            ops.flash_decode(query, k_q, k_s, k_z, vals, backend="hip")

    def test_key_page_wrong_head_dim_is_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem(dim=32)
        with pytest.raises(ValueError, match="key page"):
            ops.flash_decode(query[:, :, :16], k_q, k_s, k_z, vals, backend="hip")

    def test_scale_shape_is_checked(self):
        query, k_q, k_s, k_z, vals = _paged_problem(dim=32)
        k_s[0] = k_s[0][:5]
        with pytest.raises(ValueError, match="scale/zero-point"):
            ops.flash_decode(query, k_q, k_s, k_z, vals, backend="hip")

    def test_non_3d_query_is_rejected(self):
        query, k_q, k_s, k_z, vals = _paged_problem()
        with pytest.raises(ValueError, match="query must be"):
            ops.flash_decode(query[0], k_q, k_s, k_z, vals, backend="hip")

    def test_empty_cache_returns_exact_zeros(self):
        query, *_ = _paged_problem()
        out = ops.flash_decode(query, [], [], [], [], backend="hip")
        assert out.shape == query.shape and out.dtype == np.float32
        np.testing.assert_array_equal(out, 0.0)

    def test_lens_are_int32(self):
        query, k_q, k_s, k_z, vals = _paged_problem()
        _, lens = normalize_attention_inputs(query, k_q, k_s, k_z, vals, [64, 10, 0])
        assert lens.dtype == np.int32 and list(lens) == [64, 10, 0]
        _, lens = normalize_attention_inputs(query, k_q, k_s, k_z, vals, None)
        assert list(lens) == [64, 64, 64]


class TestBackendHonesty:
    """reference tests/test_ops_dispatch.py:90-139: a named backend is delivered or
    refused, never substituted; the package has no CPU implementation."""

    def test_unknown_backend(self):
        with pytest.raises(ValueError, match="unknown backend"):
            ops.flash_decode(*_paged_problem(), backend="nonsense")
        with pytest.raises(ValueError, match="unknown backend"):
            ops.quantize_int4(np.zeros((4, 4), np.float32), backend="nonsense")

    @pytest.mark.parametrize("name", ["reference", "triton", "pallas"])
    def test_backends_not_in_this_package_are_refused(self, name):
        with pytest.raises(ValueError):
            ops.flash_decode(*_paged_problem(), backend=name)
        with pytest.raises(ValueError):
            ops.quantize_int4(np.zeros((4, 4), np.float32), backend=name)

    def test_declared_backends(self):
        assert ops.QUANTIZE_BACKENDS == ("hip", "cuda")
        assert ops.ATTENTION_BACKENDS == ("hip", "cuda")
        assert ops.CUDA_MAX_HEAD_DIM == 256

    def test_use_cuda_false_is_refused(self):
        with pytest.raises(RuntimeError, match="CPU"):
            ops.quantize_int4(np.zeros((4, 4), np.float32), use_cuda=False)

    @pytest.mark.skipif(ops.HAS_HIP, reason="checks the no-GPU failure mode")
    def test_no_gpu_fails_loudly(self):
        with pytest.raises(RuntimeError):
            ops.quantize_int4(np.zeros((4, 4), np.float32))
        with pytest.raises(RuntimeError):
            ops.flash_decode(*_paged_problem())

    def test_backend_status(self):
        st = ops.backend_status()
        assert st["active_backend"] in ("hip", "unavailable")
        assert st["has_extension"] is True


class TestPackageExports:
    """The reference package's public names (src/__init__.py:20-56): its
    availability flags, here False because this package ships neither the
    NumPy reference functions nor a Pallas backend, and a device
    dequantize_int4 in place of dequantize_int4_ref."""

    def test_reference_flags_are_present_and_honest(self):
        import flash_decode_int4 as pkg
        assert pkg.HAS_QUANT_REF is False
        assert pkg.HAS_DECODE_REF is False
        assert pkg.HAS_PALLAS is False
        assert isinstance(pkg.HAS_CUDA, bool)
        for name in ("HAS_QUANT_REF", "HAS_DECODE_REF", "HAS_PALLAS", "HAS_CUDA",
                     "dequantize_int4", "pack_int4", "unpack_int4", "packed_nbytes"):
            assert name in pkg.__all__, name

    def test_oracle_functions_are_not_reexported(self):
        import flash_decode_int4 as pkg
        for name in ("quantize_int4_ref", "dequantize_int4_ref", "flash_decode_ref",
                     "online_softmax_ref"):
            assert not hasattr(pkg, name), name

    def test_backend_info_reports_the_flags(self, capsys):
        import flash_decode_int4 as pkg
        pkg.backend_info()
        out = capsys.readouterr().out
        assert "Quantization reference" in out and "Pallas" in out

    @pytest.mark.skipif(ops.HAS_HIP, reason="checks the no-GPU failure mode")
    def test_dequantize_without_gpu_fails_loudly(self):
        import flash_decode_int4 as pkg
        with pytest.raises(RuntimeError):
            pkg.dequantize_int4(np.zeros((2, 4), np.uint8), np.ones(4, np.float32),
                                np.zeros(4, np.float32))


class TestHostPacking:

    @pytest.mark.parametrize("shape", [(256, 64), (10, 7), (4, 128, 32), (3, 1), (1, 2)])
    def test_matches_oracle(self, shape):
        q = np.random.RandomState(shape[-1]).randint(0, 16, shape).astype(np.uint8)
        p = int4_pack.pack_int4(q)
        np.testing.assert_array_equal(p, oracle.pack_int4(q))
        np.testing.assert_array_equal(int4_pack.unpack_int4(p, shape[-1]), q)
        assert int4_pack.packed_nbytes(shape) == p.nbytes

    def test_known_answer(self):
        q = np.array([[0, 15, 15, 0, 7, 8]], dtype=np.uint8)
        np.testing.assert_array_equal(int4_pack.pack_int4(q), [[0xF0, 0x0F, 0x87]])

    def test_rejects(self):
        with pytest.raises(AssertionError):
            int4_pack.pack_int4(np.array([[16]], dtype=np.uint8))
        with pytest.raises(AssertionError):
            int4_pack.pack_int4(np.array([[1]], dtype=np.int32))


class TestWorkloads:

    def test_anchor_bytes_match_the_measurement_plan(self):
        """306,450,464 B per decode and 306,188,288 B per quantization at
        B8 x H32 x D128 x 2048 (fp32 values, 16-token pages, 128-token groups)."""
        lens = np.full(8, 2048)
        assert workloads.decode_bytes(lens, 32, 128) == 306_450_464
        assert workloads.quantize_bytes(lens, 32, 128) == 306_188_288

    @pytest.mark.parametrize("t,mb", [(512, 76.81), (8192, 1225.0), (32768, 4899.3)])
    def test_sweep_bytes(self, t, mb):
        assert abs(workloads.decode_bytes(np.full(8, t), 32, 128) / 1e6 - mb) < 0.5

    def test_cpu_workload_is_deterministic(self):
        a = workloads.make_workload("cpu")
        b = workloads.make_workload("cpu")
        for key in ("q", "k", "v_pages", "page_table", "seq_lens"):
            np.testing.assert_array_equal(a[key], b[key])
        np.testing.assert_array_equal(a["page_table"][0], np.arange(32))

    def test_page_tables_are_permutations(self):
        lens = workloads.ragged_lengths(32, 8192, 1234)
        assert lens[3] == 0 and lens[17] == 0 and (lens > 0).sum() == 30
        assert (lens % 16 != 0).any()
        table, P = workloads.page_layout(lens, 16, 1234)
        used = np.concatenate([table[b, :(lens[b] + 15) // 16] for b in range(32)])
        assert sorted(used.tolist()) == list(range(P))

    def test_rope_preserves_pair_norms(self):
        k = np.random.RandomState(0).randn(2, 10, 8).astype(np.float32)
        r = workloads.rope_rotate(k)
        n0 = k[..., :4] ** 2 + k[..., 4:] ** 2
        n1 = r[..., :4] ** 2 + r[..., 4:] ** 2
        np.testing.assert_allclose(n0, n1, rtol=1e-5)
        np.testing.assert_array_equal(r[:, 0], k[:, 0])  # position 0 is unrotated


class TestCABI:
    """The C-ABI library loads on a host without a GPU and exports every
    function include/fdi4.h declares; size queries and argument rejection run
    without touching a device."""

    def _declared(self):
        text = open(os.path.join(ROOT, "include", "fdi4.h")).read()
        return sorted(set(re.findall(r"\b(fdi4_[a-z0-9_]+)\s*\(", text)))

    def test_every_declared_symbol_is_exported(self):
        from flash_decode_int4 import capi
        lib = capi.load()
        declared = self._declared()
        assert len(declared) >= 15
        for name in declared:
            assert hasattr(lib, name), name
        assert set(declared) == set(capi.SIGNATURES), "ctypes table and header disagree"

    def test_ctypes_prototypes_match_the_header(self):
        """Parameter count and kind (pointer / int / int64 / size_t) and the
        return kind of every ctypes prototype agree with include/fdi4.h."""
        import ctypes
        from flash_decode_int4 import capi
        text = open(os.path.join(ROOT, "include", "fdi4.h")).read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        protos = re.findall(r"([A-Za-z_][\w\s\*]*?)\b(fdi4_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;",
                            text, flags=re.S)

        def kind_c(decl):
            decl = " ".join(decl.split())
            if "*" in decl or "hipStream_t" in decl:
                return "ptr"
            base = decl.replace("const ", "").split()[0]
            return {"int": "int", "int32_t": "int", "int64_t": "int64",
                    "size_t": "size_t"}[base]

        def kind_py(t):
            if t in (ctypes.c_void_p, ctypes.c_char_p) or hasattr(t, "_type_") and \
                    isinstance(getattr(t, "_type_"), type):
                return "ptr"
            return {ctypes.c_int: "int", ctypes.c_int32: "int", ctypes.c_int64: "int64",
                    ctypes.c_size_t: "size_t"}[t]

        assert {name for _, name, _ in protos} == set(capi.SIGNATURES)
        for ret, name, params in protos:
            params = " ".join(params.split())
            c_args = [] if params in ("", "void") else [kind_c(p) for p in params.split(",")]
            res, args = capi.SIGNATURES[name]
            assert [kind_py(a) for a in args] == c_args, name
            assert kind_py(res) == kind_c(ret.split("extern")[-1]), name

    def test_only_declared_symbols_are_exported(self):
        """Internal helpers stay out of the library's dynamic symbol table."""
        import shutil
        import subprocess
        from flash_decode_int4 import capi
        nm = shutil.which("nm")
        if nm is None:
            pytest.skip("nm not available")
        out = subprocess.run([nm, "-D", "--defined-only", capi.LIB_PATH],
                             capture_output=True, text=True, check=True).stdout
        names = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
        public = {n for n in names if not n.startswith("_")}
        assert public == set(self._declared())

    def test_size_queries(self):
        from flash_decode_int4 import capi
        lib = capi.load()
        assert lib.fdi4_abi_version() == 1
        assert lib.fdi4_quantize_rows_workspace_bytes(512, 128) == (2 * 128 + 128) * 8
        assert lib.fdi4_decode_workspace_bytes(8, 32, 128, 1) == 0
        n = 8 * 32 * 4
        assert lib.fdi4_decode_workspace_bytes(8, 32, 128, 4) == n * 128 * 4 + n * 16
        assert lib.fdi4_decode_partials_bytes(8, 32, 128, 1) == 8 * 32 * (512 + 16)
        # B8 x H32 (one q-head per kv-head), float32 values: 4-wave
        # workgroups, one wave per SIMD, one split and no merge; float16
        # values: 8-wave workgroups, one split.
        for v_dtype in (capi.V_F32, capi.V_F16):
            cache = capi.PagedCache(max_pages=128, page_rows=16, num_kv_heads=32, head_dim=128,
                                    v_dtype=v_dtype)
            assert lib.fdi4_decode_num_splits(8, 32, cache) == 1
            # T=512 (32 chunks): still one split.
            cache = capi.PagedCache(max_pages=32, page_rows=16, num_kv_heads=32, head_dim=128,
                                    v_dtype=v_dtype)
            assert lib.fdi4_decode_num_splits(8, 32, cache) == 1
        # B1 x H8 x 32768 tokens: 2048 chunks split 32 ways (1024 waves of
        # four-wave workgroups with float32 values, 2048 of eight with float16).
        for v_dtype in (capi.V_F32, capi.V_F16):
            cache = capi.PagedCache(max_pages=2048, page_rows=16, num_kv_heads=8, head_dim=128,
                                    v_dtype=v_dtype)
            assert lib.fdi4_decode_num_splits(1, 8, cache) == 32
        # B1 x H8 x 1024 tokens (64 chunks): at least 4 chunks per wave, so
        # four splits of four-wave workgroups (float32 values), two of eight.
        cache = capi.PagedCache(max_pages=64, page_rows=16, num_kv_heads=8, head_dim=128)
        assert lib.fdi4_decode_num_splits(1, 8, cache) == 4
        cache = capi.PagedCache(max_pages=64, page_rows=16, num_kv_heads=8, head_dim=128,
                                v_dtype=capi.V_F16)
        assert lib.fdi4_decode_num_splits(1, 8, cache) == 2
        # GQA B8 x Hq32 x Hkv8 at D=128: four q-heads per workgroup, so 64
        # workgroups of 8 waves and 4 splits for ~2048 waves.
        cache = capi.PagedCache(max_pages=512, page_rows=16, num_kv_heads=8, head_dim=128)
        assert lib.fdi4_decode_num_splits(8, 32, cache) == 4

    def test_invalid_arguments_are_rejected_before_any_device_call(self):
        _run_with_no_gpu("check_invalid_arguments_are_rejected")

    def test_typed_decode_rejects_unknown_element_types(self):
        _run_with_no_gpu("check_typed_decode_rejects_unknown_element_types")

    def test_tuning_knobs_are_explicit_and_validated(self):
        """Launch-shape overrides go through fdi4_set_tuning (the library
        reads no environment); out-of-range values are refused and leave the
        knob unchanged; the context manager restores the previous values."""
        from flash_decode_int4 import capi
        lib = capi.load()
        for knob in capi.TUNE.values():
            assert lib.fdi4_get_tuning(knob) == 0
        assert lib.fdi4_get_tuning(99) == -1 and lib.fdi4_set_tuning(99, 1) == 1
        waves = capi.TUNE["decode_waves"]
        assert lib.fdi4_set_tuning(waves, 6) == 1 and lib.fdi4_get_tuning(waves) == 0
        with capi.tuning(decode_waves=4, decode_heads_per_wg=2):
            assert lib.fdi4_get_tuning(waves) == 4
            assert lib.fdi4_get_tuning(capi.TUNE["decode_heads_per_wg"]) == 2
            cache = capi.PagedCache(max_pages=32, page_rows=16, num_kv_heads=32, head_dim=128,
                                    v_dtype=capi.V_F16)
            # 4 waves x 8 chunks each: B8 H32 with float16 values now needs two
            # splits for ~2048 waves.
            assert lib.fdi4_decode_num_splits(8, 32, cache) == 2
        assert lib.fdi4_get_tuning(waves) == 0
        with pytest.raises(ValueError):
            capi.tuning(decode_wave=4)
        with pytest.raises(RuntimeError):
            with capi.tuning(decode_vector_only=2):
                pass
        text = open(os.path.join(ROOT, "int4-kv-cache-quantization-cuda-triton-pallas_amd",
                                 "csrc", "capi.hip")).read()
        assert "getenv" not in text


# The rejection checks pass fake device addresses to calls that are otherwise
# valid. On a host with a GPU they run in a child process that sees none, so a
# host check that regressed makes the call fail there instead of launching a
# kernel on those addresses.

_CHILD = """
import ctypes, sys
sys.path[:0] = {paths!r}
hip = ctypes.CDLL("libamdhip64.so")
n = ctypes.c_int(-1)
rc = hip.hipGetDeviceCount(ctypes.byref(n))
if rc == 0 and n.value > 0:
    print("SKIP: a GPU is still visible with HIP_VISIBLE_DEVICES/ROCR_VISIBLE_DEVICES hidden")
    sys.exit(0)
import importlib.util
spec = importlib.util.spec_from_file_location("host_contract_child", {path!r})
mod = importlib.util.module_from_spec(spec)
spec.loader.exec_module(mod)
mod.{fn}()
print("PASS")
"""


def _run_with_no_gpu(fn_name):
    import subprocess
    import sys
    import torch
    if torch.cuda.device_count() == 0:       # counting does not initialize a device
        globals()[fn_name]()
        return
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1",
               CUDA_VISIBLE_DEVICES="-1")
    paths = [ROOT, os.path.join(ROOT, "tests"),
             os.path.join(ROOT, "int4-kv-cache-quantization-cuda-triton-pallas_amd")]
    code = _CHILD.format(paths=paths, path=os.path.abspath(__file__), fn=fn_name)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    if "SKIP:" in r.stdout:
        pytest.skip(r.stdout.strip())
    assert "PASS" in r.stdout, r.stdout + r.stderr


def check_invalid_arguments_are_rejected():
    from flash_decode_int4 import capi
    lib = capi.load()
    bad = 1  # hipErrorInvalidValue
    assert lib.fdi4_quantize_rows(None, 4, 4, 4, None, 4, 0, None, None, None, 0, None) == bad
    assert lib.fdi4_decode_paged(None, 1, 1, 0, 0, None, None, 0, 0, 0, None, 0, None) == bad
    cache = capi.PagedCache(head_dim=96, page_rows=16, num_kv_heads=1, pages_per_group=1,
                            max_pages=1, num_pages=1, k_pages=16, k_scale=16, k_zp=16)
    assert lib.fdi4_quantize_paged(16, 1, 16, 0, 0, 128, 128, cache, None) == bad
    assert lib.fdi4_merge_splits(None, None, 1, 1, 128, 1, None, 0, 0, None) == bad
    assert lib.fdi4_flash_decode_int4_ws(None, None, None, None, None, None, 1, 1, 300, 1, 1,
                                         None, None, 0, None) == bad
    # Row strides whose 16-row chunk does not fit in 31 bits of byte
    # offset (the kernels address a chunk's rows with 32-bit offsets).
    big = capi.PagedCache(head_dim=128, page_rows=16, num_kv_heads=1, pages_per_group=8,
                          max_pages=8, num_pages=8, k_pages=256, k_scale=256, k_zp=256,
                          k_page_stride=1 << 30, k_row_stride=1 << 27,
                          v_pages=256, v_dtype=capi.V_F32, v_page_stride=1 << 12,
                          v_row_stride=128, s_group_stride=128, seq_lens=256)
    q = ctypes.c_void_p(256)
    assert lib.fdi4_decode_paged(q, 1, 1, 128, 128, ctypes.byref(big), q, 128, 128, 1,
                                 None, 0, None) == bad
    big.k_row_stride = 64
    big.v_row_stride = 1 << 25
    assert lib.fdi4_decode_paged(q, 1, 1, 128, 128, ctypes.byref(big), q, 128, 128, 1,
                                 None, 0, None) == bad
    # Sequences of 2^32 token positions (max_pages x page_rows) do not fit
    # the kernels' 32-bit token indices.
    big.v_row_stride = 128
    big.page_rows, big.max_pages, big.pages_per_group = 32, 1 << 27, 4
    big.page_table, big.pt_batch_stride = 256, 1 << 27
    assert lib.fdi4_decode_paged(q, 1, 1, 128, 128, ctypes.byref(big), q, 128, 128, 1,
                                 None, 0, None) == bad
    assert lib.fdi4_append_paged(q, 128, 128, q, 128, 128, 1, q, 1 << 14, 1 << 14, 128,
                                 128, ctypes.byref(big), None) == bad
    # Split partials larger than the no-allocation decode's static array
    # (B64 x Hq64 x 2 splits at D=256: 8 MiB + 128 KiB) are refused.
    wide = capi.PagedCache(head_dim=256, page_rows=16, num_kv_heads=64, pages_per_group=8,
                           max_pages=8, num_pages=8, k_pages=256, k_scale=256, k_zp=256,
                           k_page_stride=1 << 16, k_head_stride=1 << 10, k_row_stride=128,
                           v_pages=256, v_dtype=capi.V_F32, v_page_stride=1 << 20,
                           v_head_stride=1 << 12, v_row_stride=256, s_batch_stride=1 << 17,
                           s_head_stride=1 << 11, s_group_stride=256, seq_lens=256)
    # The serving-step pair: the second lengths array must be given, must not
    # overlap the cache's lengths, and the cache must carry lengths.
    ok = capi.PagedCache(head_dim=128, page_rows=16, num_kv_heads=1, pages_per_group=8,
                         max_pages=8, num_pages=8, k_pages=256, k_scale=256, k_zp=256,
                         k_page_stride=1024, k_row_stride=64, v_pages=256, v_dtype=capi.V_F32,
                         v_page_stride=2048, v_row_stride=128, s_group_stride=128,
                         seq_lens=1024)
    for lens_other in (None, 1024, 1028, 1020):   # missing, same array, overlapping
        assert lib.fdi4_decode_paged_advance(q, 0, 2, 1, 128, 128, ctypes.byref(ok), q, 0, 128,
                                             128, 1, None, 0, lens_other, None) == bad
        assert lib.fdi4_append_paged_advance(q, 128, 128, q, 128, 128, 2, q, 1 << 14, 1 << 14,
                                             128, 128, ctypes.byref(ok), lens_other,
                                             None) == bad
    ok.seq_lens = None
    assert lib.fdi4_decode_paged_advance(q, 0, 2, 1, 128, 128, ctypes.byref(ok), q, 0, 128,
                                         128, 1, None, 0, 4096, None) == bad
    assert lib.fdi4_decode_workspace_bytes(64, 64, 256, 2) > capi.NOALLOC_SCRATCH_BYTES
    assert lib.fdi4_decode_paged_noalloc(q, 64, 64, 1 << 14, 256, ctypes.byref(wide), q,
                                         1 << 14, 256, 2, None) == bad
    # Dequantization: missing pointers, rows shorter than the channels they
    # hold (unpacked and packed), negative scale strides.
    assert lib.fdi4_dequantize_int4(None, 4, 8, 8, 0, q, q, 0, 1, q, 8, None) == bad
    assert lib.fdi4_dequantize_int4(q, 4, 8, 8, 0, q, None, 0, 1, q, 8, None) == bad
    assert lib.fdi4_dequantize_int4(q, 4, 8, 7, 0, q, q, 0, 1, q, 8, None) == bad
    assert lib.fdi4_dequantize_int4(q, 4, 9, 4, 1, q, q, 0, 1, q, 9, None) == bad
    assert lib.fdi4_dequantize_int4(q, 4, 8, 8, 0, q, q, 0, 1, q, 7, None) == bad
    assert lib.fdi4_dequantize_int4(q, 4, 8, 8, 0, q, q, -1, 1, q, 8, None) == bad
    assert lib.fdi4_dequantize_int4(q, 4, 0, 8, 0, q, q, 0, 1, q, 8, None) == bad
    # Zero rows: nothing to do, no device call.
    assert lib.fdi4_dequantize_int4(None, 0, 8, 8, 0, None, None, 0, 1, None, 8, None) == 0


def check_typed_decode_rejects_unknown_element_types():
    """fdi4_decode_paged_ex: query and output types are 0, 1, 2 (float32,
    float16, bfloat16); value pages fp32, fp16 or bf16; anything else is
    refused before any device call."""
    from flash_decode_int4 import capi
    lib = capi.load()
    bad = 1
    ok_cache = capi.PagedCache(head_dim=128, page_rows=16, num_kv_heads=1, pages_per_group=8,
                               max_pages=8, num_pages=8, k_pages=256, k_scale=256, k_zp=256,
                               k_page_stride=1024, k_row_stride=64, v_pages=256,
                               v_dtype=capi.V_BF16, v_page_stride=2048, v_row_stride=128,
                               s_group_stride=128, seq_lens=256)
    q = ctypes.c_void_p(256)
    for q_dtype, o_dtype in ((3, 0), (0, 3), (-1, 1), (2, 7)):
        assert lib.fdi4_decode_paged_ex(q, q_dtype, 1, 1, 128, 128, ctypes.byref(ok_cache),
                                        q, o_dtype, 128, 128, 1, None, 0, None) == bad
    ok_cache.v_dtype = 3
    assert lib.fdi4_decode_paged_ex(q, 1, 1, 1, 128, 128, ctypes.byref(ok_cache), q, 1,
                                    128, 128, 1, None, 0, None) == bad
    assert capi.V_BF16 == 2 and capi.K_BF16 == 2

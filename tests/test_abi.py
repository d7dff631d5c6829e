"""C-ABI checks that need no GPU: the library loads, exports every symbol the
headers declare, the ctypes struct matches the C layout, and argument errors are
reported with the right status before any device call (no context needed)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from pcp_amd import _lib
from pcp_amd._lib import DType, PcpError
from pcp_amd.backend import HipGrpoBackend, execute_raw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = []
    for h in sorted(os.listdir(INCLUDE)):
        if not h.endswith(".h"):
            continue
        with open(os.path.join(INCLUDE, h)) as f:
            text = f.read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(pcp_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (pcp_\w+)", out))
    assert set(names) <= exported


@pytest.mark.parametrize("cname,pyty", [("pcp_grpo_args", _lib.GrpoArgs), ("pcp_lmhead_args", _lib.LmheadArgs)])
def test_struct_layout_matches_c(tmp_path, cname, pyty):
    fields = [f[0] for f in pyty._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", '#include "pcp_grpo.h"', "int main(void){",
           f'printf("%zu\\n", sizeof({cname}));']
    src += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    src += ["return 0;}"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", INCLUDE, str(c), "-o", str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(pyty)
    for f, off in zip(fields, vals[1:]):
        assert getattr(pyty, f).offset == off, f


def test_c_host_links_against_the_library(tmp_path):
    # A C caller (what a Zig @cImport binding compiles to) links and runs without a GPU.
    src = r'''
#include <stdio.h>
#include "pcp_grpo.h"
int main(void) {
  pcp_grpo_args a; pcp_grpo_args_init(&a);
  a.n_seq = 0;
  int rc = pcp_grpo_loss_fwd_bwd(NULL, &a);
  printf("%d %s|%s\n", rc, pcp_last_error(NULL), pcp_version());
  return 0;
}'''
    c = tmp_path / "host.c"
    c.write_text(src)
    exe = tmp_path / "host"
    libdir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run(["gcc", "-std=c99", "-I", INCLUDE, str(c), "-L", libdir, "-lpcp_grpo", f"-Wl,-rpath,{libdir}",
                    "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    assert out.startswith("-1 n_seq must be >= 1") and "gfx950" in out


def test_args_defaults():
    a = _lib.default_args()
    assert a.logits_dtype == DType.bf16 and a.ids_dtype == DType.i64 and a.mask_dtype == DType.f32
    assert abs(a.clip_eps - 0.2) < 1e-7 and abs(a.kl_beta - 0.04) < 1e-8 and abs(a.std_eps - 1e-8) < 1e-15
    assert a.group_size == 1 and a.loss_norm == 0 and a.flags == 0


def _valid_args():
    a = _lib.default_args()
    a.n_seq, a.rows, a.vocab, a.group_size = 2, 4, 16, 2
    a.logits = 0x1000
    a.ids = 0x2000
    a.advantages = 0x3000
    return a


@pytest.mark.parametrize("mutate,code,text", [
    (lambda a: setattr(a, "n_seq", 0), -1, "n_seq"),
    (lambda a: setattr(a, "vocab", 0), -1, "vocab"),
    (lambda a: setattr(a, "vocab", (1 << 31) - (1 << 20) + 1), -1, "2^31 - 2^20"),
    (lambda a: setattr(a, "group_size", 0), -1, "group_size"),
    (lambda a: setattr(a, "logit_seq_stride", 3), -1, "logit_seq_stride"),
    (lambda a: setattr(a, "tok_offset", 1), -1, "tok_offset"),
    (lambda a: setattr(a, "logits_dtype", int(DType.i32)), -2, "logits dtype"),
    (lambda a: setattr(a, "ids_dtype", int(DType.f32)), -2, "ids dtype"),
    (lambda a: (setattr(a, "mask", 0x10), setattr(a, "mask_dtype", int(DType.i64))), -2, "mask dtype"),
    (lambda a: setattr(a, "logits", None), -1, "logits is NULL"),
    (lambda a: setattr(a, "ids", None), -1, "ids is NULL"),
    (lambda a: setattr(a, "logits", 0x1001), -1, "element size"),
    (lambda a: (setattr(a, "logits_dtype", int(DType.f32)), setattr(a, "logits", 0x1002)), -1, "element size"),
    (lambda a: (setattr(a, "ref_logits", 0x4001), setattr(a, "loss_mode", 1)), -1, "element size"),
    (lambda a: (setattr(a, "dlogits", 0x5002), setattr(a, "dlogits_dtype", int(DType.f32))), -1, "element size"),
    (lambda a: setattr(a, "loss_mode", 7), -1, "loss_mode"),
    (lambda a: setattr(a, "loss_mode", 1), -1, "ref_logits"),
    (lambda a: setattr(a, "advantages", None), -1, "both NULL"),
    (lambda a: setattr(a, "clip_eps", 1.5), -1, "clip_eps"),
    (lambda a: (setattr(a, "dlogits", 0x10), setattr(a, "dlogits_dtype", int(DType.f16))), -2, "dlogits dtype"),
    (lambda a: (setattr(a, "n_seq", 1 << 40), setattr(a, "rows", 1 << 20)), -9, "2^31"),
])
def test_argument_errors_without_device(mutate, code, text):
    L = _lib.lib()
    a = _valid_args()
    mutate(a)
    rc = L.pcp_grpo_loss_fwd_bwd(None, ctypes.byref(a))
    assert rc == code
    assert text in L.pcp_last_error(None).decode()


def _valid_lm_args():
    a = _lib.LmheadArgs()
    _lib.lib().pcp_lmhead_args_init(ctypes.byref(a))
    a.n_seq, a.rows, a.hidden, a.vocab = 2, 4, 128, 1000
    a.hidden_states, a.weight, a.ids, a.rewards = 0x1000, 0x2000, 0x3000, 0x4000
    return a


def test_lmhead_args_defaults():
    a = _valid_lm_args()
    assert a.group_size == 1 and a.ids_dtype == DType.i64 and a.mask_dtype == DType.f32 and a.vocab_chunk == 0
    assert abs(a.clip_eps - 0.2) < 1e-7 and abs(a.kl_beta - 0.04) < 1e-8 and a.loss_mode == 0
    assert abs(a.norm_eps - 1e-6) < 1e-12 and not a.norm_weight and not a.dnorm_weight


@pytest.mark.parametrize("mutate,code,text", [
    (lambda a: setattr(a, "hidden", 96), -1, "multiple of 64"),
    (lambda a: setattr(a, "vocab_chunk", 100), -1, "vocab_chunk"),
    (lambda a: setattr(a, "weight", None), -1, "is NULL"),
    (lambda a: setattr(a, "weight", 0x2008), -1, "16-byte aligned"),
    (lambda a: setattr(a, "ids_dtype", int(DType.f32)), -2, "ids dtype"),
    (lambda a: setattr(a, "loss_mode", 1), -1, "ref_weight"),
    (lambda a: setattr(a, "rewards", None), -1, "both NULL"),
    (lambda a: (setattr(a, "n_seq", 1 << 20), setattr(a, "rows", 1 << 10)), -9, "2^28"),
    (lambda a: setattr(a, "dnorm_weight", 0x5000), -1, "needs norm_weight"),
    (lambda a: (setattr(a, "norm_weight", 0x5000), setattr(a, "hidden", 8256)), -1, "hidden <= 8192"),
    (lambda a: (setattr(a, "norm_weight", 0x5000), setattr(a, "norm_eps", float("nan"))), -1, "norm_eps"),
])
def test_lmhead_argument_errors_without_device(mutate, code, text):
    L = _lib.lib()
    a = _valid_lm_args()
    mutate(a)
    assert L.pcp_grpo_lmhead_fwd_bwd(None, ctypes.byref(a)) == code
    assert text in L.pcp_last_error(None).decode()
    b = _valid_lm_args()
    assert L.pcp_grpo_lmhead_fwd_bwd(None, ctypes.byref(b)) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()


def test_noalloc_rejects_oversized_requests_without_device():
    # The allocation-free entry point checks its work space against the static array
    # before it needs a context: 2^20 + 1 per-token losses do not fit in 4 MiB.
    a = _valid_args()
    a.rows = (1 << 20) + 1
    rc = _lib.lib().pcp_grpo_loss_fwd_bwd_noalloc(None, ctypes.byref(a))
    assert rc == -9
    assert b"allocation-free" in _lib.lib().pcp_last_error(None)
    a.rows = 4
    rc = _lib.lib().pcp_grpo_loss_fwd_bwd_noalloc(None, ctypes.byref(a))
    assert rc == -1 and b"context is NULL" in _lib.lib().pcp_last_error(None)


def test_noalloc_rejects_an_oversized_live_row_list_without_device():
    # Without zero-fill the live-row list (4 bytes per logits row) also lives in the
    # array: with the per-token losses passed in, 2^20 + 1 rows of list alone do not fit,
    # while the same request with zero-fill (no list) passes the size check.
    a = _valid_args()
    a.n_seq, a.rows, a.group_size = 1, (1 << 20) + 1, 1
    a.dlogits, a.token_loss = 0x4000, 0x5000
    a.flags = _lib.FLAG_NO_ZERO_FILL
    rc = _lib.lib().pcp_grpo_loss_fwd_bwd_noalloc(None, ctypes.byref(a))
    assert rc == -9
    assert b"allocation-free" in _lib.lib().pcp_last_error(None)
    a.flags = 0
    rc = _lib.lib().pcp_grpo_loss_fwd_bwd_noalloc(None, ctypes.byref(a))
    assert rc == -1 and b"context is NULL" in _lib.lib().pcp_last_error(None)


def test_workspace_calls_without_device():
    L = _lib.lib()
    assert L.pcp_release_workspace(None) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()
    assert L.pcp_workspace_bytes(None) == 0


def test_valid_args_then_null_context():
    L = _lib.lib()
    a = _valid_args()
    assert L.pcp_grpo_loss_fwd_bwd(None, ctypes.byref(a)) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()


def test_init_rejects_other_backends_and_reports_missing_device():
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.pcp_init(int(_lib.Backend.cuda), 0, ctypes.byref(h)) == -10
    if not torch.cuda.is_available():
        with pytest.raises(PcpError) as e:
            HipGrpoBackend.init(_lib.Backend.rocm, 0)
        assert e.value.code == -6


def _ref_inputs(S=2, T=5, V=11, ids=None):
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((S, T, V)).astype(np.float32)
    ids = rng.integers(0, V, (S, T)).astype(np.int64) if ids is None else ids
    mask = np.ones((S, T), np.float32)
    adv = np.array([1.0, -1.0], np.float32)[:S]
    return [logits, ids, mask, adv], [logits.shape, ids.shape, mask.shape, adv.shape]


def test_execute_argument_errors_without_device():
    data, shapes = _ref_inputs()
    dts = [DType.f32, DType.i64, DType.f32, DType.f32]
    with pytest.raises(PcpError) as e:
        execute_raw(None, "no_such_fn", data, shapes, dts)
    assert e.value.code == -7
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_loss_fwd_bwd", data[:3], shapes[:3], dts[:3])
    assert e.value.code == -8
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_loss_fwd_bwd", data, [shapes[0], (2, 4), shapes[2], shapes[3]], dts)
    assert e.value.code == -1   # byte count does not match the shape
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_loss_fwd_bwd", data, shapes, [DType.f64, DType.i64, DType.f32, DType.f32])
    assert e.value.code == -1   # f64 bytes != f32 bytes for the same shape -> size mismatch first
    bad = np.array(data[0], np.float64)
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_loss_fwd_bwd", [bad] + data[1:], shapes, [DType.f64, DType.i64, DType.f32, DType.f32])
    assert e.value.code == -2
    ids = data[1].copy()
    ids[1, 3] = 11                  # == V: out of range
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_loss_fwd_bwd", [data[0], ids, data[2], data[3]], shapes, dts)
    assert e.value.code == -3
    ids[1, 3] = -100                # the ignore index is accepted
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_loss_fwd_bwd", [data[0], ids, data[2], data[3]], shapes, dts)
    assert e.value.code == -1 and "context is NULL" in str(e.value)
    # dtypes == NULL selects the function's defaults (f32 / i64)
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_loss_fwd_bwd", data, shapes, None)
    assert "context is NULL" in str(e.value)


def test_execute_main_names_the_split():
    # The reference's "main" is the whole training step (params in, parameter gradients
    # out); the library holds its loss head only and says how to split the VMFB.
    data, shapes = _ref_inputs()
    with pytest.raises(PcpError) as e:
        execute_raw(None, "main", data, shapes, [DType.f32, DType.i64, DType.f32, DType.f32])
    assert e.value.code == -10
    msg = str(e.value)
    assert "grpo_loss_fwd_bwd" in msg and "forward to logits" in msg and "backward seeded with dlogits" in msg
    with pytest.raises(PcpError) as e:
        HipGrpoBackend(None, _lib.Backend.rocm, 0).executeTrainingStep(None, data, shapes)
    assert e.value.code == -10


def _lm_inputs(S=2, T=6, H=64, V=40):
    rng = np.random.default_rng(1)
    hidden = rng.integers(0, 1 << 16, (S, T, H)).astype(np.uint16)
    w = rng.integers(0, 1 << 16, (V, H)).astype(np.uint16)
    ids = rng.integers(0, V, (S, T)).astype(np.int64)
    mask = np.ones((S, T), np.float32)
    old = np.zeros((S, T), np.float32)
    rewards = np.array([1.0, 0.0], np.float32)[:S]
    hyper = np.array([S, 0.2, 0.04, 0, 1], np.float32)
    data = [hidden, w, w, ids, mask, old, rewards, hyper]
    dts = [DType.bf16, DType.bf16, DType.bf16, DType.i64, DType.f32, DType.f32, DType.f32, DType.f32]
    return data, [x.shape for x in data], dts


def test_execute_lmhead_argument_errors_without_device():
    data, shapes, dts = _lm_inputs()
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data[:7], shapes[:7], dts[:7])
    assert e.value.code == -8
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data, shapes, [DType.f16] + dts[1:])
    assert e.value.code == -2 and "hidden" in str(e.value)
    bad_w = data[1][:, :32].copy()
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", [data[0], bad_w] + data[2:], [shapes[0], bad_w.shape] + shapes[2:], dts)
    assert e.value.code == -1 and "weight" in str(e.value)
    hyper = data[7].copy()
    hyper[4] = 3
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data[:7] + [hyper], shapes, dts)
    assert e.value.code == -1 and "loss_mode" in str(e.value)
    ids = data[3].copy()
    ids[0, 0] = 999                 # position 0 is never a target under the shift: accepted
    ids[1, 2] = 40                  # == V at a target position: rejected
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data[:3] + [ids] + data[4:], shapes, dts)
    assert e.value.code == -3
    ids[1, 2] = 0
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data[:3] + [ids] + data[4:], shapes, dts)
    assert e.value.code == -1 and "context is NULL" in str(e.value)
    # the optional ninth input (final norm weight): its shape, its dtype, hyper of 6
    gamma = np.ones(64, np.float32)
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data + [gamma[:32]], shapes + [(32,)], dts + [DType.f32])
    assert e.value.code == -1 and "norm_weight" in str(e.value)
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data + [gamma.view(np.int32)], shapes + [(64,)], dts + [DType.i32])
    assert e.value.code == -2 and "norm_weight" in str(e.value)
    hyper6 = np.append(data[7], np.float32(1e-5))
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data[:7] + [hyper6], shapes[:7] + [(6,)], dts)
    assert e.value.code == -1 and "hyper" in str(e.value)     # six entries only with the norm
    with pytest.raises(PcpError) as e:
        execute_raw(None, "grpo_lmhead_fwd_bwd", data[:7] + [hyper6, gamma], shapes[:7] + [(6,), (64,)],
                    dts + [DType.f32])
    assert e.value.code == -1 and "context is NULL" in str(e.value)


def test_philox_known_answers():
    # Random123 known-answer vectors for philox4x32-10.
    from pcp_amd.synth import philox
    assert philox([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert philox([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert philox([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]) == \
        [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_step_api_argument_errors_without_device():
    L = _lib.lib()
    h = ctypes.c_void_p()
    counts = (ctypes.c_int64 * 3)(4, 5, 6)
    assert L.pcp_nesterov_create(None, 0.1, 0.9, 7, 3, counts, ctypes.byref(h)) == -1
    assert "mode" in L.pcp_last_error(None).decode()
    assert L.pcp_nesterov_create(None, 0.1, 0.9, 0, 0, counts, ctypes.byref(h)) == -1
    neg = (ctypes.c_int64 * 2)(3, -1)
    assert L.pcp_nesterov_create(None, 0.1, 0.9, 0, 2, neg, ctypes.byref(h)) == -1
    assert L.pcp_nesterov_create(None, float("nan"), 0.9, 0, 3, counts, ctypes.byref(h)) == -1
    assert L.pcp_nesterov_create(None, 0.1, 0.9, 0, 3, counts, ctypes.byref(h)) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode() and not h.value
    assert L.pcp_nesterov_update(None, 0, None, None, 0, None) == -1
    assert L.pcp_nesterov_update_flat(None, None, None, None, None) == -1
    assert L.pcp_nesterov_reset(None, None) == -1
    assert L.pcp_nesterov_total(None) == -1
    assert L.pcp_nesterov_serialize(None, None, 0) == -1
    assert L.pcp_nesterov_deserialize(None, None, 0) == -1
    L.pcp_nesterov_destroy(None)
    st = _lib.GradStats()
    assert L.pcp_grad_stats_compute(None, None, 5, 0, ctypes.byref(st), None) == -1
    assert L.pcp_grad_stats_compute(None, None, 0, 0, ctypes.byref(st), None) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()
    assert L.pcp_pack_rollouts(None, None, 0, None, None, 0, None, 3, 2, 8, 0x10, 0x20, None) == -1
    assert "n_rollouts <= n_rows" in L.pcp_last_error(None).decode()
    assert L.pcp_pack_rollouts(None, None, 0, 0x10, None, 0, 0x20, 1, 2, 8, 0x10, 0x20, None) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()
    assert L.pcp_pack_rollouts(None, None, 0, 0x10, None, 0, 0x20, 1, 1 << 40, 1 << 30, 0x10, 0x20, None) == -9


def test_grad_stats_struct_layout(tmp_path):
    fields = [f[0] for f in _lib.GradStats._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", '#include "pcp_step.h"', "int main(void){",
           'printf("%zu\\n", sizeof(pcp_grad_stats));']
    src += [f'printf("%zu\\n", offsetof(pcp_grad_stats, {f}));' for f in fields]
    src += ["return 0;}"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", INCLUDE, str(c), "-o", str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(_lib.GradStats)
    for f, off in zip(fields, vals[1:]):
        assert getattr(_lib.GradStats, f).offset == off, f


def test_sampler_argument_errors_without_device():
    L = _lib.lib()
    assert L.pcp_sample_tokens(None, 0x1000, int(DType.f16), 4, 100, 100, 1.0, 0x2000, 0x3000, None) == -2
    assert L.pcp_sample_tokens(None, 0x1000, int(DType.f32), 4, 100, 50, 1.0, 0x2000, 0x3000, None) == -1
    assert L.pcp_sample_tokens(None, 0x1000, int(DType.f32), 4, (1 << 20) + 1, (1 << 20) + 4, 1.0, 0x2000,
                               0x3000, None) == -1
    assert L.pcp_sample_tokens(None, 0x1008, int(DType.f32), 4, 100, 100, 1.0, 0x2000, 0x3000, None) == -1
    assert "16-byte" in L.pcp_last_error(None).decode()
    assert L.pcp_sample_tokens(None, 0x1000, int(DType.f32), 4, 100, 100, 1.0, None, 0x3000, None) == -1
    assert "uniforms" in L.pcp_last_error(None).decode()
    assert L.pcp_sample_tokens(None, 0x1000, int(DType.f32), 4, 100, 100, 0.0, None, 0x3000, None) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()     # greedy needs no uniforms


def _write_prompts(path, prompts):
    import struct
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(prompts)))
        for p in prompts:
            f.write(struct.pack("<I", len(p)))
            for t in p:
                f.write(struct.pack("<Q", t))


def test_prompt_file_counts_and_errors_without_device(tmp_path):
    """The .bin of tools/prepare_rl_dataset.py:28-40, written here with struct as that
    script does, read back by the library (counting pass, no device)."""
    from pcp_amd import formats
    p = tmp_path / "prompts.bin"
    _write_prompts(p, [[1, 2, 3], [], [151935, 7]])
    assert formats.prompt_counts(str(p)) == (3, 5)
    raw = p.read_bytes()
    (tmp_path / "cut.bin").write_bytes(raw[:-3])                # ends inside the last prompt
    with pytest.raises(PcpError) as e:
        formats.prompt_counts(str(tmp_path / "cut.bin"))
    assert e.value.code == -13
    with pytest.raises(PcpError) as e:
        formats.prompt_counts(str(tmp_path / "missing.bin"))
    assert e.value.code == -14
    _write_prompts(tmp_path / "big.bin", [[1 << 63]])           # the reference's @intCast to i64 fails
    with pytest.raises(PcpError) as e:
        formats.prompt_counts(str(tmp_path / "big.bin"))
    assert e.value.code == -9


def test_weights_and_base64_errors_without_device(tmp_path):
    L = _lib.lib()
    w = tmp_path / "w.bin"
    w.write_bytes(np.arange(10, dtype=np.float32).tobytes())
    counts = (ctypes.c_int64 * 2)(6, 5)                         # 11 floats > 10 in the file
    assert L.pcp_weights_load(None, str(w).encode(), 2, counts, 0x1000, None) == -13
    assert "WeightFileTooSmall" in L.pcp_last_error(None).decode()
    assert L.pcp_weights_load(None, str(tmp_path / "no.bin").encode(), 2, counts, 0x1000, None) == -14
    ok = (ctypes.c_int64 * 2)(6, 4)
    assert L.pcp_weights_load(None, str(w).encode(), 2, ok, 0x1000, None) == -1   # valid: needs a context
    assert "context is NULL" in L.pcp_last_error(None).decode()
    assert [L.pcp_base64_encoded_len(n) for n in (0, 1, 2, 3, 4, 5, 6)] == [0, 4, 4, 4, 8, 8, 8]
    n = ctypes.c_int64()
    assert L.pcp_base64_decode(None, 0x1000, 6, 0x2000, ctypes.byref(n), None) == -1
    assert "multiple of 4" in L.pcp_last_error(None).decode()


def test_hbm_stream_argument_errors_without_device():
    """pcp_hbm_stream rejects a bad kind or shape, a size off 16 bytes, NULL or misaligned
    buffers before any device work (the context check comes after them)."""
    L = _lib.lib()
    assert L.pcp_hbm_stream(None, 4, 0, 1, 0x1000, 0x2000, 0x3000, 1 << 20, None) == -1
    assert "kind" in L.pcp_last_error(None).decode()
    assert L.pcp_hbm_stream(None, 2, 0, 3, 0x1000, None, 0x3000, 1 << 20, None) == -1
    assert "vectors_per_lane" in L.pcp_last_error(None).decode()
    assert L.pcp_hbm_stream(None, 2, 0, 1, 0x1000, None, 0x3000, 1000, None) == -1
    assert L.pcp_hbm_stream(None, 3, 1, 1, 0x1000, None, 0x3000, 1 << 20, None) == -1
    assert "NULL" in L.pcp_last_error(None).decode()
    assert L.pcp_hbm_stream(None, 2, 0, 1, 0x1008, None, 0x3000, 1 << 20, None) == -1
    assert L.pcp_hbm_stream(None, 0, 0, 1, 0x1000, None, None, 1 << 20, None) == -1
    assert L.pcp_hbm_stream(None, 1, 0, 8, None, None, 0x3000, 1 << 20, None) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()
    # 64 GiB at one vector per lane is 2^32 lanes: rejected before any launch; at two
    # vectors per lane the same size passes the checks (and stops at the NULL context).
    assert L.pcp_hbm_stream(None, 1, 0, 1, None, None, 0x3000, 1 << 36, None) == -1
    assert "2^32 lanes" in L.pcp_last_error(None).decode()
    assert L.pcp_hbm_stream(None, 1, 0, 2, None, None, 0x3000, 1 << 36, None) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()


def test_mfma_peak_argument_errors_without_device():
    """pcp_mfma_peak rejects a bad shape or grid, odd or too few rounds, a NULL or
    misaligned buffer before any device work (the context check comes after them)."""
    L = _lib.lib()
    assert L.pcp_mfma_peak(None, 2, 1, 2, 0, 0x1000, None, None) == -1
    assert "shape" in L.pcp_last_error(None).decode()
    assert L.pcp_mfma_peak(None, 0, 0, 2, 0, 0x1000, None, None) == -1
    assert "workgroups" in L.pcp_last_error(None).decode()
    assert L.pcp_mfma_peak(None, 1, 1, 3, 0, 0x1000, None, None) == -1
    assert L.pcp_mfma_peak(None, 0, 1, 0, 0, 0x1000, None, None) == -1
    assert L.pcp_mfma_peak(None, 0, 1, 2, 0, None, None, None) == -1
    assert "NULL" in L.pcp_last_error(None).decode()
    assert L.pcp_mfma_peak(None, 1, 1, 2, 0, 0x1002, None, None) == -1
    assert L.pcp_mfma_peak(None, 0, 1, 2, 0, 0x1000, 0x2004, None) == -1
    assert L.pcp_mfma_peak(None, 1, 1, 2, 0, 0x1000, 0x2000, None) == -1
    assert "context is NULL" in L.pcp_last_error(None).decode()


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits with status 2 and a JSON line that says this
    build runs on one GPU (before it touches a device)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    p = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], cwd=root,
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 2, (p.returncode, p.stderr[-500:])
    assert "one GPU only" in p.stdout

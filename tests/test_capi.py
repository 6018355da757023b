"""C ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments (with MLX-style messages) before any
HIP call is made. Mirrors the error path higgs relies on
(crates/higgs-models/src/qwen3_next.rs:552-576: status != 0 plus a message)."""
import os
import re
import threading

import pytest
import torch

from higgs_amd import _lib, ops
from higgs_amd._lib import HiggsQmmError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "higgs_qmm.h")
FAKE = 0x7F0000000000  # never dereferenced: validation fails before any launch


def header_symbols():
    txt = open(HEADER).read()
    return set(re.findall(r"^(?:const\s+)?(?:char\s*\*|int|void)\s*\*?\s*(hq_\w+)\s*\(", txt, re.M))


def test_exports_every_header_symbol():
    syms = header_symbols()
    assert {"hq_quantized_matmul", "hq_gather_qmm", "hq_dequantize", "hq_last_error",
            "hq_version", "hq_result_dtype", "hq_embedding_dequantize"} <= syms
    L = _lib.lib()
    for s in syms:
        assert hasattr(L, s), s
    assert set(_lib.SIGNATURES) == syms


def test_per_width_code_is_not_shared_between_widths():
    """Each kernel source is compiled once per bit width; any symbol those
    builds share (weak, merged by the linker) must carry the width as its
    first template argument, or one width's code would serve all of them."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-C", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    shared = [ln.split(" ", 2)[2] for ln in out.splitlines()
              if len(ln.split(" ", 2)) == 3 and ln.split(" ", 2)[1] in ("W", "V")
              and "hq::" in ln]
    assert shared, "expected the per-width kernel instantiations"
    pat = re.compile(r"^void hq::(?:__device_stub__)?\w+_kernel<[2-8], ")
    bad = [sym for sym in shared if not pat.match(sym)]
    assert not bad, bad[:10]


def test_version_and_result_dtype():
    assert "gfx950" in _lib.version()
    L = _lib.lib()
    F32, F16, BF16 = 0, 1, 2
    table = {(F32, F32): F32, (F16, F16): F16, (BF16, BF16): BF16, (BF16, F16): F32,
             (F16, BF16): F32, (F32, BF16): F32, (BF16, F32): F32}
    for (a, b), r in table.items():
        assert L.hq_result_dtype(a, b) == r
    assert L.hq_result_dtype(3, 0) == -1


def qmm(**kw):
    a = dict(y=FAKE, x=FAKE, w=FAKE, s=FAKE, b=FAKE, M=1, N=64, K=128, transpose=1, g=64,
             bits=4, xdt=2, sdt=2)
    a.update(kw)
    return _lib.lib().hq_quantized_matmul(a["y"], a["x"], a["w"], a["s"], a["b"], a["M"],
                                          a["N"], a["K"], a["transpose"], a["g"], a["bits"],
                                          a["xdt"], a["sdt"], None)


@pytest.mark.parametrize("kw,needle", [
    (dict(bits=7), "bits 7 is not supported"),
    (dict(bits=1), "bits 1 is not supported"),
    (dict(g=16), "group size 16 is not supported"),
    (dict(K=96), "divisible by the group size"),
    (dict(transpose=0, N=100, g=64), "divisible by the group size"),
    (dict(xdt=7), "floating"),
    (dict(sdt=-1), "floating"),
    (dict(M=-1), "Invalid sizes"),
    (dict(K=0), "Invalid sizes"),
    (dict(y=0), "NULL"),
    (dict(w=0), "NULL"),
    (dict(x=FAKE + 8), "16-byte aligned"),
])
def test_quantized_matmul_rejects(kw, needle):
    rc = qmm(**kw)
    assert rc == _lib.HQ_ERR_INVALID_ARGUMENT
    assert needle in _lib.last_error()


def test_empty_calls_succeed_without_gpu():
    assert qmm(M=0) == 0
    assert qmm(N=0) == 0
    L = _lib.lib()
    assert L.hq_gather_qmm(FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 0, 1, 4, 1, 64, 128, 1, 64,
                           4, 1, 2, 2, None) == 0
    assert L.hq_dequantize(FAKE, FAKE, FAKE, FAKE, 0, 128, 64, 4, 2, None) == 0
    assert L.hq_embedding_dequantize(FAKE, FAKE, FAKE, FAKE, None, 0, 10, 128, 64, 4, 2,
                                     None) == 0


def test_gather_rejects():
    L = _lib.lib()

    def call(lhs=None, rhs=FAKE, batch=8, xb=8, wb=4, bits=4, g=64):
        return L.hq_gather_qmm(FAKE, FAKE, FAKE, FAKE, FAKE, lhs, rhs, batch, xb, wb, 1, 64, 128,
                               1, g, bits, 1, 2, 2, None)

    assert call(rhs=None) == 1 and "rhs_indices" in _lib.last_error()
    assert call(batch=6, xb=4) == 1 and "multiple of x's batch" in _lib.last_error()
    assert call(wb=0) == 1 and "Invalid sizes" in _lib.last_error()
    assert call(bits=9) == 1


def test_dequantize_rejects():
    L = _lib.lib()
    assert L.hq_dequantize(FAKE, FAKE, FAKE, FAKE, 4, 100, 64, 4, 2, None) == 1
    assert "multiple of the group" in _lib.last_error()
    assert L.hq_dequantize(FAKE + 4, FAKE, FAKE, FAKE, 4, 128, 64, 4, 2, None) == 1
    assert L.hq_embedding_dequantize(FAKE, FAKE, FAKE, FAKE, None, 3, 10, 128, 64, 4, 2,
                                     None) == 1
    assert "indices" in _lib.last_error()


def test_last_error_is_thread_local():
    assert qmm(bits=7) == 1
    seen = []
    t = threading.Thread(target=lambda: seen.append(_lib.last_error()))
    t.start()
    t.join()
    assert seen == [""]
    assert "bits 7" in _lib.last_error()


# --- host facade validation (mirrors MLX's messages; CPU tensors suffice) ----

def _q(N=64, K=128, bits=4, g=64, lead=()):
    w = torch.zeros((*lead, N, K * bits // 32), dtype=torch.int32)
    s = torch.zeros((*lead, N, K // g), dtype=torch.bfloat16)
    return w, s, s.clone()


def test_facade_shape_errors():
    w, s, b = _q()
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    with pytest.raises(HiggsQmmError, match="Scales and biases should have the same shape"):
        ops.quantized_matmul(x, w, s, b[:, :1])
    with pytest.raises(HiggsQmmError, match="incompatible based on bits and group_size"):
        ops.quantized_matmul(x, w, s, b, group_size=32)
    with pytest.raises(HiggsQmmError, match="does not match the expanded quantized matrix"):
        ops.quantized_matmul(torch.zeros(1, 64, dtype=torch.bfloat16), w, s, b)
    with pytest.raises(HiggsQmmError, match="should be uint32"):
        ops.quantized_matmul(x, w.float(), s, b)
    with pytest.raises(HiggsQmmError, match="bits 7 is not supported"):
        ops.quantized_matmul(x, w, s, b, bits=7)
    with pytest.raises(HiggsQmmError, match="Only real floating types"):
        ops.quantized_matmul(x.to(torch.int32), w, s, b)
    with pytest.raises(HiggsQmmError, match="must live on the GPU"):
        ops.quantized_matmul(x, w, s, b)
    with pytest.raises(HiggsQmmError, match="Shape of scales and biases does not match"):
        ops.dequantize(w, s[:, :1], b[:, :1])
    with pytest.raises(HiggsQmmError, match="at least two dimensions"):
        ops.gather_qmm(x[0], w, s, b, rhs_indices=torch.zeros(1, dtype=torch.int32))


def test_prefix_broadcast_rule():
    pb = ops._prefix_broadcast
    assert pb((2, 3, 1), (2, 3, 8))      # forward_gather: x [B,L,1] vs idx [B,L,k]
    assert pb((4096,), (4096,))          # global sort: one x row per index
    assert pb((1,), (7,)) and pb((), (7,))
    assert not pb((3,), (2, 3))          # x broadcast along a leading dim
    assert not pb((1, 3), (2, 3))


# --- fused SwiGLU and MoE entry points: validation before any launch ---------

def swiglu_mm(**kw):
    a = dict(h=FAKE, x=FAKE, wg=FAKE, sg=FAKE, bg=FAKE, wu=FAKE, su=FAKE, bu=FAKE, M=1, N=64,
             K=1024, g=64, bits=4, xdt=2, sdt=2)
    a.update(kw)
    return _lib.lib().hq_quantized_matmul_swiglu(
        a["h"], a["x"], a["wg"], a["sg"], a["bg"], a["wu"], a["su"], a["bu"], a["M"], a["N"],
        a["K"], a["g"], a["bits"], a["xdt"], a["sdt"], None)


@pytest.mark.parametrize("kw,code,needle", [
    (dict(bits=7), 1, "bits 7 is not supported"),
    (dict(K=96), 1, "divisible by the group size"),
    (dict(wu=0), 1, "NULL"),
    (dict(h=FAKE + 4), 1, "16-byte aligned"),
    (dict(xdt=0, sdt=0), 2, "one 16-bit dtype"),
    (dict(xdt=2, sdt=1), 2, "one 16-bit dtype"),
    (dict(M=3, K=768), 2, "K % 1024 == 0"),
    (dict(M=300, K=97 * 32, g=32), 2, "K % 64 == 0"),
])
def test_quantized_matmul_swiglu_rejects(kw, code, needle):
    assert swiglu_mm(**kw) == code
    assert needle in _lib.last_error()


def test_swiglu_entry_empty_and_shape_errors():
    assert swiglu_mm(M=0) == 0 and swiglu_mm(N=0) == 0
    L = _lib.lib()
    assert L.hq_swiglu(FAKE, FAKE, FAKE, 0, 2, None) == 0
    assert L.hq_swiglu(FAKE, FAKE, FAKE, 16, 5, None) == 1 and "floating" in _lib.last_error()
    assert L.hq_swiglu(FAKE, FAKE, FAKE, -1, 2, None) == 1
    assert L.hq_gather_qmm_swiglu(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, 4,
                                  4, 2, 1, 64, 128, 64, 4, 2, 2, None) == 1
    assert "rhs_indices" in _lib.last_error()
    assert L.hq_gather_qmm_swiglu(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 6,
                                  4, 2, 1, 64, 128, 64, 4, 2, 2, None) == 1
    assert "multiple of x's batch" in _lib.last_error()


def test_moe_sort_and_combine_reject():
    L = _lib.lib()
    assert L.hq_moe_sort(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 8, 128, None) == 0
    assert L.hq_moe_sort(FAKE, FAKE, FAKE, FAKE, FAKE, 64, 8, 4096, None) == 1
    assert "num_experts <= 2048" in _lib.last_error()
    assert L.hq_moe_sort(FAKE, FAKE, FAKE, FAKE, FAKE, 64, 0, 128, None) == 1
    assert L.hq_moe_sort(FAKE, FAKE, FAKE, FAKE, None, 64, 8, 128, None) == 1
    assert "idx" in _lib.last_error()
    assert L.hq_moe_combine(FAKE, FAKE, FAKE, FAKE, 0, 8, 2048, 2, 2, None) == 0
    assert L.hq_moe_combine(FAKE, FAKE, FAKE, FAKE, 4, 8, 2048, 9, 2, None) == 1
    assert L.hq_moe_combine(FAKE, FAKE, None, FAKE, 4, 8, 2048, 2, 2, None) == 1
    assert "NULL" in _lib.last_error()
    assert L.hq_moe_combine(FAKE + 2, FAKE, FAKE, FAKE, 4, 8, 2048, 2, 2, None) == 1
    assert "aligned" in _lib.last_error()


# --- quantized_linear (bias epilogue) and quantize: validation before launch --

def qlin(**kw):
    a = dict(y=FAKE, x=FAKE, w=FAKE, s=FAKE, b=FAKE, lb=FAKE, M=1, N=64, K=128, g=64, bits=4,
             xdt=2, sdt=2, bdt=2)
    a.update(kw)
    return _lib.lib().hq_quantized_linear(a["y"], a["x"], a["w"], a["s"], a["b"], a["lb"],
                                          a["M"], a["N"], a["K"], a["g"], a["bits"], a["xdt"],
                                          a["sdt"], a["bdt"], None)


@pytest.mark.parametrize("kw,code,needle", [
    (dict(bits=7), 1, "bits 7 is not supported"),
    (dict(K=96), 1, "divisible by the group size"),
    (dict(bdt=9), 1, "the bias has dtype code 9"),
    (dict(bdt=0), 2, "must be the output dtype"),            # bf16 product, f32 bias
    (dict(xdt=2, sdt=1, bdt=2), 2, "must be the output dtype"),  # mixed -> f32 output
    (dict(y=0), 1, "NULL"),
    (dict(x=FAKE + 2), 1, "16-byte aligned"),
])
def test_quantized_linear_rejects(kw, code, needle):
    assert qlin(**kw) == code
    assert needle in _lib.last_error()


def test_quantized_linear_without_bias_ignores_its_dtype():
    # a NULL bias is plain quantized_matmul: the bias dtype code is not read
    assert qlin(lb=None, bdt=9, M=0) == 0
    assert qlin(lb=None, bdt=9, bits=7) == 1 and "bits 7" in _lib.last_error()


def quant(**kw):
    a = dict(wq=FAKE, s=FAKE, b=FAKE, w=FAKE, rows=4, K=128, g=64, bits=4, dt=2)
    a.update(kw)
    return _lib.lib().hq_quantize(a["wq"], a["s"], a["b"], a["w"], a["rows"], a["K"], a["g"],
                                  a["bits"], a["dt"], None)


@pytest.mark.parametrize("kw,needle", [
    (dict(bits=1), "bits 1 is not supported"),
    (dict(g=48), "group size 48 is not supported"),
    (dict(K=96), "divisible by the group size"),
    (dict(K=0), "divisible by the group size"),
    (dict(rows=-1), "divisible by the group size"),
    (dict(dt=5), "floating"),
    (dict(wq=0), "NULL"),
    (dict(w=FAKE + 8), "16-byte aligned"),
    (dict(wq=FAKE + 2), "4-byte aligned"),
    (dict(dt=0, s=FAKE + 2), "float32 scales and biases must be 4-byte aligned"),
])
def test_quantize_rejects(kw, needle):
    assert quant(**kw) == _lib.HQ_ERR_INVALID_ARGUMENT
    assert needle in _lib.last_error()


def test_quantize_empty_succeeds_without_gpu():
    assert quant(rows=0) == 0


def test_facade_quantize_and_linear_errors():
    w, s, b = _q()
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    with pytest.raises(HiggsQmmError, match="must have shape"):
        ops.quantized_linear(x, w, s, b, torch.zeros(3, dtype=torch.bfloat16))
    with pytest.raises(HiggsQmmError, match="must be the output dtype"):
        ops.quantized_linear(x, w, s, b, torch.zeros(64, dtype=torch.float32))
    with pytest.raises(HiggsQmmError, match="divisible by the quantization group size"):
        ops.quantize(torch.zeros(4, 96), 64, 4)
    with pytest.raises(HiggsQmmError, match="Only real floating types can be quantized"):
        ops.quantize(torch.zeros(4, 128, dtype=torch.int32), 64, 4)
    with pytest.raises(HiggsQmmError, match="must live on the GPU"):
        ops.quantize(torch.zeros(4, 128), 64, 4)


def test_switch_projection_settings():
    """Each SwitchLinear projection may carry its own (group_size, bits)."""
    t3 = (1, 2, 3)
    assert ops._proj(t3, 64, 4) == ((1, 2, 3), 64, 4)
    assert ops._proj((1, 2, 3, 32, 8), 64, 4) == ((1, 2, 3), 32, 8)
    with pytest.raises(HiggsQmmError):
        ops._proj((1, 2), 64, 4)



def test_grouped_stream_kernel_waits_for_its_lds_dma():
    """The streaming grouped kernel (hq_gqms.hip) loads x straight into LDS,
    issues the first weight tile's loads behind it, and then waits with an
    explicit vmcnt of exactly those weight loads before the barrier, so the
    weights stay in flight. That is only correct if the code from the last LDS
    DMA to the barrier is straight-line and holds that many vector-memory
    instructions; check every instantiation in the compiled gfx950 assembly."""
    import shutil
    import subprocess
    import tempfile

    from higgs_amd import build as hb

    if shutil.which(hb.HIPCC) is None and not os.path.exists(hb.HIPCC):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as td:
        asm = os.path.join(td, "gqms.s")
        subprocess.run([hb.HIPCC, *hb.FLAGS, "-DHQ_BITS=4", "--cuda-device-only", "-S",
                        os.path.join(hb.CSRC, "hq_gqms.hip"), "-o", asm],
                       check=True, capture_output=True)
        txt = open(asm).read()
    kernels = re.split(r"\n(_ZN\S*gqms_kernel\S+):", txt)[1:]
    assert kernels, "no gqms_kernel instantiation in the assembly"
    vm_op = re.compile(r"^\s+(global_|buffer_|scratch_|flat_)")
    for name, body in zip(kernels[0::2], kernels[1::2]):
        lines = body.split("\n")
        dmas = [i for i, ln in enumerate(lines) if "global_load_lds" in ln]
        assert dmas, name
        # from the last DMA, one straight run ending in the waited barrier
        # (DMAs of unused row slots before it may be skipped)
        last = dmas[-1]
        bar = next(i for i in range(last, len(lines)) if re.match(r"^\s+s_barrier", lines[i]))
        span = lines[last:bar]
        assert not any(re.match(r"^\S+:", ln) or re.match(r"^\s+s_(c)?branch", ln)
                       for ln in span), name
        between = [ln for ln in lines[last + 1:bar] if vm_op.match(ln)]
        waits = [ln for ln in lines[last + 1:bar] if "s_waitcnt" in ln and "vmcnt" in ln]
        assert waits, name
        vm = int(re.search(r"vmcnt\((\d+)\)", waits[-1]).group(1))
        assert vm == len(between) > 0, (name, vm, len(between))

"""torch.ops.leankv: every registered overload has a Meta kernel giving the GPU op's output shapes and dtypes.

Runs on the CPU (meta tensors carry no data, no kernel launches).  The GPU
implementations are exercised against the oracle in tests/test_gpu_ops.py.
"""

import torch

import leankv_amd.kernels as K

F16, F32, U8, I32 = torch.float16, torch.float32, torch.uint8, torch.int32


def _e(*shape, dt=F16):
    return torch.empty(*shape, dtype=dt, device="meta")


def _calls():
    o = torch.ops.leankv
    x, w = _e(4096), _e(1024, 4096)
    X, Pi, b, c = _e(2, 8, 10, 128, dt=F32), _e(128, 128, dt=F32), _e(7, dt=F32), _e(8, dt=F32)
    kc, kn, hot = _e(1, 8, 100, 64, dt=U8), _e(1, 8, 100, dt=F32), _e(1, 8, 64, 128)
    q1, qp, seq = _e(1, 32, 128), _e(1, 32, 5, 128), _e(1, dt=I32)
    attn = (kc, kn, kc, kn, hot, hot, Pi, Pi, c, 3)
    return {
        "sparse_gemv": (lambda: o.sparse_gemv(x, w, 0.1), [((1024,), F16)]),
        "sparse_gemv.out": (lambda: o.sparse_gemv.out(x, w, 0.1, out=_e(1024)), [((1024,), F16)]),
        "sparse_gateup_swiglu": (lambda: o.sparse_gateup_swiglu(x, w, w, 0.1, 0.2), [((1024,), F16)]),
        "sparse_gateup_swiglu.out": (lambda: o.sparse_gateup_swiglu.out(x, w, w, 0.1, 0.2, out=_e(1024)),
                                     [((1024,), F16)]),
        "sparse_qkv": (lambda: o.sparse_qkv(x, _e(4096, 4096), w, w, 0.1, 0.1, 0.1),
                       [((4096,), F16), ((1024,), F16), ((1024,), F16)]),
        "sparse_qkv.out": (lambda: o.sparse_qkv.out(x, w, w, w, 0., 0., 0., q=_e(1024), k=_e(1024), v=_e(1024)),
                           [((1024,), F16)] * 3),
        "tq_quantize": (lambda: o.tq_quantize(X, Pi, b, 3), [((2, 8, 10, 64), U8), ((2, 8, 10), F32)]),
        "tq_quantize_rotated": (lambda: o.tq_quantize_rotated(X, b, 3), [((2, 8, 10, 64), U8)]),
        "tq_dequantize": (lambda: o.tq_dequantize(kc, kn, Pi, c, 3, F16), [((1, 8, 100, 128), F16)]),
        "tq_rotate": (lambda: o.tq_rotate(X.half(), Pi, True), [((2, 8, 10, 128), F32)]),
        "rms_norm": (lambda: o.rms_norm(_e(3, 4096), _e(4096), 1e-5), [((3, 4096), F16)]),
        "tq_cache_append": (lambda: o.tq_cache_append(_e(8, 128), _e(8, 128), hot, hot, kc, kn, kc, kn, Pi, Pi, b, 3,
                                                      seq), []),
        "tq_decode_attn": (lambda: o.tq_decode_attn(q1, *attn, seq, 164, 0.1), [((1, 32, 128), F16)]),
        "tq_decode_attn.out": (lambda: o.tq_decode_attn.out(q1, *attn, seq, 164, 0.1, out=_e(1, 32, 128)),
                               [((1, 32, 128), F16)]),
        "tq_prefill_attn": (lambda: o.tq_prefill_attn(qp, *attn, 164, 0.1), [((1, 32, 5, 128), F16)]),
        "tq_prefill_attn.out": (lambda: o.tq_prefill_attn.out(qp, *attn, 164, 0.1, out=_e(1, 32, 5, 128)),
                                [((1, 32, 5, 128), F16)]),
    }


def test_every_op_has_a_meta_kernel():
    calls = _calls()
    assert sorted(calls) == sorted(K.op_names())
    for name, (fn, want) in calls.items():
        out = fn()
        outs = [] if out is None else (list(out) if isinstance(out, (tuple, list)) else [out])
        got = [(tuple(t.shape), t.dtype) for t in outs]
        assert got == want, (name, got, want)


def test_out_overloads_return_the_given_buffer():
    o = torch.ops.leankv
    out = _e(1024)
    assert o.sparse_gemv.out(_e(4096), _e(1024, 4096), 0.1, out=out) is out

"""Weights read from a GGUF file through the library's reader feed the GEMV
on the GPU: the tensors a Q4_K_M decode multiplies at batch 1 (Q4_K FFN
gate/up, Q6_K FFN down and output projection, Mistral-7B shapes), written to
a GGUF file with the test writer, mapped by q4k_gguf_open, uploaded and
multiplied; results equal the in-memory weights' results bit for bit and the
oracle's within the parity tolerance."""
import numpy as np
import pytest

import _common
import gguf_writer as W

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_q4_k_m_layer_from_gguf(Q, O, gpu, tmp_path):
    K, F = 4096, 14336
    up = Q.quantize_rows_q4_K(_common.weights(F, K, seed=1), nthreads=16)
    gate = Q.quantize_rows_q4_K(_common.weights(F, K, seed=2), nthreads=16)
    down = Q.quantize_rows_q6_K(_common.weights(K, F, seed=3), nthreads=16)
    out = Q.quantize_rows_q6_K(_common.weights(2048, K, seed=4), nthreads=16)  # an output-projection slice
    path = tmp_path / "layer.gguf"
    W.write_gguf(path, [("general.architecture", W.STRING, "llama"), ("general.file_type", W.UINT32, 15)],
                 [("blk.0.ffn_up.weight", 12, [K, F], up.tobytes()), ("blk.0.ffn_gate.weight", 12, [K, F], gate.tobytes()),
                  ("blk.0.ffn_down.weight", 14, [F, K], down.tobytes()), ("output.weight", 14, [K, 2048], out.tobytes())])
    x = _common.activations(1, K, seed=5)
    with Q.GGUFFile(str(path)) as g:
        assert g.metadata()["general.file_type"] == 15
        tu = to_dev(g.weight_rows("blk.0.ffn_up.weight"), gpu)
        tg = to_dev(g.weight_rows("blk.0.ffn_gate.weight"), gpu)
        td = to_dev(g.weight_rows("blk.0.ffn_down.weight"), gpu)
        to = to_dev(g.weight_rows("output.weight"), gpu)
        types = {n: t["type"] for n, t in g.tensors.items()}
    xd = to_dev(x, gpu)
    # gate/up fused with SWIGLU, then the down projection of the result
    h = Q.mul_mat_vec_q_fused(tu, K, xd, gate=tg, glu_op=Q.GLU_OP_SWIGLU, wtype=types["blk.0.ffn_up.weight"])
    y = Q.mul_mat_vec_q(td, F, h, wtype=types["blk.0.ffn_down.weight"]).cpu().numpy()
    # the same from the in-memory weights
    h2 = Q.mul_mat_vec_q_fused(to_dev(up, gpu), K, xd, gate=to_dev(gate, gpu), glu_op=Q.GLU_OP_SWIGLU)
    y2 = Q.mul_mat_vec_q(to_dev(down, gpu), F, h2, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    assert np.array_equal(y, y2)
    # oracle on the down projection of the GPU's h
    ref = O.gemv_q6K_q8_1(down, F, O.quantize_q8_1(h.cpu().numpy()), want_sums=False)
    _common.assert_within_tolerance(O, y, ref, "ffn_down from GGUF")
    yo = Q.mul_mat_vec_q(to, K, xd, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    refo = O.gemv_q6K_q8_1(out, K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, yo, refo, "output from GGUF")

"""GPU parity: ``W4A16Linear`` (reference w4a16-kernel/src/w4a16/linear.py)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import DEV, assert_gemm_close, log, np_
from oracle import w4a16_oracle as O

pytestmark = pytest.mark.gpu


def test_w4a16_linear_end_to_end():
    """Reference test_correctness.py:73-89 (K=N=4096, M=16, seed 2), checked against
    the oracle's linear forward on the module's own buffers."""
    from w4a16 import W4A16Linear

    log("linear end-to-end")
    torch.manual_seed(2)
    K, N, M = 4096, 4096, 16
    lin = torch.nn.Linear(K, N, bias=True).to(DEV).half()
    qlin = W4A16Linear.from_linear(lin, group_size=128)
    x = torch.randn(M, K, dtype=torch.float16, device=DEV)
    y = qlin(x)
    assert y.shape == (M, N)
    ref = O.linear_forward(np_(x), np_(qlin.qweight), np_(qlin.scales), np_(qlin.zeros),
                           np_(qlin.bias), 128)
    assert_gemm_close(y, ref, "W4A16Linear")


def test_from_linear_quantises_transpose_bit_exact():
    """from_linear transposes nn.Linear's [N, K] weight (linear.py:66) before
    quantising; buffers equal the oracle's quantisation of weight.T."""
    from w4a16 import W4A16Linear

    log("from_linear buffers")
    torch.manual_seed(3)
    lin = torch.nn.Linear(512, 384, bias=False).half()
    qlin = W4A16Linear.from_linear(lin, group_size=64)      # CPU module, GPU compute
    assert qlin.qweight.device.type == "cpu" and qlin.bias is None
    rq, rs, rz = O.quantize_weight(lin.weight.detach().t().contiguous().numpy(), 64)
    assert np.array_equal(qlin.qweight.numpy(), rq)
    assert np.array_equal(qlin.scales.numpy().view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(qlin.zeros.numpy().view(np.uint16), rz.view(np.uint16))


@pytest.mark.parametrize("shape", [(2, 3, 1024), (1, 1024), (5, 1, 1024)])
def test_forward_leading_dims_and_state_dict(shape):
    from w4a16 import W4A16Linear

    log(f"linear leading dims {shape}")
    torch.manual_seed(4)
    lin = torch.nn.Linear(1024, 260, bias=True).to(DEV).half()
    qlin = W4A16Linear.from_linear(lin, group_size=128)
    x = torch.randn(*shape, dtype=torch.float16, device=DEV)
    y = qlin(x)
    assert y.shape == (*shape[:-1], 260)
    ref = O.linear_forward(np_(x), np_(qlin.qweight), np_(qlin.scales), np_(qlin.zeros),
                           np_(qlin.bias), 128)
    assert_gemm_close(y.reshape(-1, 260), ref.reshape(-1, 260), "leading dims")
    # state_dict round trip into a fresh module gives identical output
    fresh = W4A16Linear(1024, 260, group_size=128, device=DEV)
    fresh.load_state_dict(qlin.state_dict())
    assert torch.equal(fresh(x), y)


def test_forward_any_input_layout():
    """forward takes x in any layout the reference accepts (it reshapes and
    copies to contiguous rows): a row-strided column slice runs in place (the
    kernels take rows >= K apart), a transposed view and a broadcast row
    (stride 0) are copied first; all give the contiguous input's bits."""
    from w4a16 import W4A16Linear

    log("linear input layouts")
    torch.manual_seed(5)
    lin = torch.nn.Linear(512, 132, bias=True).to(DEV).half()
    qlin = W4A16Linear.from_linear(lin, group_size=64)
    wide = torch.randn(6, 640, dtype=torch.float16, device=DEV)
    for what, x in (("column slice", wide[:, 64:576]),
                    ("transposed", wide[:, :512].t().contiguous().t()),
                    ("broadcast row", wide[:1, :512].expand(6, 512)),
                    ("3-d slice", wide.view(2, 3, 640)[..., 100:612])):
        y = qlin(x)
        assert torch.equal(y, qlin(x.contiguous())), what
        ref = O.linear_forward(np_(x.reshape(-1, 512)), np_(qlin.qweight), np_(qlin.scales),
                               np_(qlin.zeros), np_(qlin.bias), 64)
        assert_gemm_close(y.reshape(-1, 132), ref, what)

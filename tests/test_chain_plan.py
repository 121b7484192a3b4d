"""CPU checks of the decode-chain planner (include/gq_chain.h): what it
accepts and refuses, and the workspace it asks for.  No GPU is used: the
planner's validation and sizing run on the host."""
import ctypes

import pytest

import gq


class _T:
    """Stands in for a device tensor: the planner only reads addresses."""

    def __init__(self, addr):
        self.addr = addr

    def data_ptr(self):
        return self.addr


def _op(n, k, **kw):
    o = {"w": _T(0x10000), "x": _T(0x20000), "y": _T(0x30000), "N": n, "K": k}
    o.update(kw)
    return o


def layer_ops(base=0):
    """q, k, v, o, gate/up, down of a Llama-3-8B layer as chain ops."""
    d = lambda *ix: [base + i for i in ix]  # noqa: E731
    return [_op(4096, 4096, gamma=_T(1), deps=d(-1 - base) if base else []),
            _op(1024, 4096, gamma=_T(1)),
            _op(1024, 4096, gamma=_T(1)),
            _op(4096, 4096, x_head_dim=128, x_group=4, resid=_T(2), deps=d(0, 1, 2)),
            _op(14336, 4096, w_up=_T(3), gamma=_T(1), deps=d(3)),
            _op(4096, 14336, resid=_T(4), deps=d(4))]


def test_chain_plan_sizes_a_decode_step():
    ops = layer_ops()
    n = gq.chain_workspace_bytes(gq.FMT_Q4_K, ops)
    # completion flags (one word per op and workgroup, 256 workgroups at
    # most), error flag and the op table: one device op per op (down's 14336
    # columns are within one op's K range)
    ws = lambda ops: 256 + 4 * 256 * ops + 256 + 256 * ((ops * 128 + 255) // 256)  # noqa: E731
    assert n == ws(6)
    assert gq.chain_workspace_bytes(gq.FMT_Q4_0, ops) == n
    assert gq.chain_workspace_bytes(gq.FMT_Q8_0, ops) == n
    assert gq.chain_workspace_bytes(gq.FMT_Q8_0, [_op(128256, 4096, gamma=_T(1))]) == ws(1)
    # K beyond one op's range (16384) is cut into column ranges chained
    # through the residual: 40960 columns -> 3 device ops
    assert gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 40960)]) == ws(3)


@pytest.mark.parametrize("bad", [
    lambda: [_op(64, 256, deps=[0])],                                 # a dependency on itself
    lambda: [_op(64, 256), _op(64, 256, deps=[2])],                   # on a later op
    lambda: [_op(64, 100)],                                           # K not a multiple of 32
    lambda: [_op(64, 256, w_up=_T(5), resid=_T(6))],                  # SwiGLU with a residual
    lambda: [_op(64, 32768, gamma=_T(1))],                            # a cut op cannot normalise
    lambda: [_op(64, 20480, w_up=_T(5))],                             # nor be a SwiGLU pair
    lambda: [_op(64, 256, x_head_dim=12, x_group=2)],                 # GQA runs of 8
    lambda: [_op(64, 512, k_offset=128, k_total=1024)],               # range not on a chunk (Q4_K: 256)
])
def test_chain_plan_refuses(bad):
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, bad())


def test_chain_plan_refuses_formats():
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q6_K, [_op(64, 256)])

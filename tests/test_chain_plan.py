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


_next = [0x100000]


def _buf(nfloats=1 << 18):
    """A distinct, 256-byte aligned fake device address range."""
    a = _next[0]
    _next[0] += (4 * nfloats + 255) // 256 * 256
    return _T(a)


def _op(n, k, **kw):
    o = {"w": _buf(), "x": _buf(), "y": _buf(), "N": n, "K": k}
    o.update(kw)
    return o


def layer_ops(base=0, h_in=None, h_out=None):
    """q, k, v, o, gate/up, down of a Llama-3-8B layer as chain ops, with the
    data flow of a decode step: q/k/v read h_in, o reads v through the GQA map
    and adds h_in, gate/up read h1, down reads act and adds h1."""
    d = lambda *ix: [base + i for i in ix]  # noqa: E731
    h_in = h_in or _buf()
    h_out = h_out or _buf()
    an, fn, q, k, v, h1, act = (_buf(16384) for _ in range(7))
    prev = d(-1) if base else []
    return [_op(4096, 4096, x=h_in, gamma=an, y=q, deps=prev),
            _op(1024, 4096, x=h_in, gamma=an, y=k, deps=prev),
            _op(1024, 4096, x=h_in, gamma=an, y=v, deps=prev),
            _op(4096, 4096, x=v, x_head_dim=128, x_group=4, resid=h_in, y=h1, deps=d(0, 1, 2)),
            _op(14336, 4096, w_up=_buf(), x=h1, gamma=fn, y=act, deps=d(3)),
            _op(4096, 14336, x=act, resid=h1, y=h_out, deps=d(4))]


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
    assert gq.chain_workspace_bytes(gq.FMT_Q8_0, [_op(128256, 4096, gamma=_buf())]) == ws(1)
    # K beyond one op's range (16384) is cut into column ranges chained
    # through the residual: 40960 columns -> 3 device ops
    assert gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 40960)]) == ws(3)


@pytest.mark.parametrize("bad", [
    lambda: [_op(64, 256, deps=[0])],                                 # a dependency on itself
    lambda: [_op(64, 256), _op(64, 256, deps=[2])],                   # on a later op
    lambda: [_op(64, 100)],                                           # K not a multiple of 32
    lambda: [_op(64, 256, w_up=_buf(), resid=_buf())],                  # SwiGLU with a residual
    lambda: [_op(64, 32768, gamma=_buf())],                            # a cut op cannot normalise
    lambda: [_op(64, 20480, w_up=_buf())],                             # nor be a SwiGLU pair
    lambda: [_op(64, 256, x_head_dim=12, x_group=2)],                 # GQA runs of 8
    lambda: [_op(64, 512, k_offset=128, k_total=1024)],               # range not on a chunk (Q4_K: 256)
    lambda: [_op(64, 256, x=_T(0x100004))],                           # x not 16-byte aligned
    lambda: [_op(64, 256, gamma=_T(0x100008))],                       # gamma not 16-byte aligned
    lambda: [_op(64, 256, y=_T(0x100002))],                           # y not 4-byte aligned
    lambda: [_op(64, 256, resid=_T(0x100001))],                       # resid not 4-byte aligned
])
def test_chain_plan_refuses(bad):
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, bad())


def test_chain_plan_refuses_formats():
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q6_K, [_op(64, 256)])


def test_chain_plan_write_hazards():
    """An op that overwrites what an earlier op reads or writes must depend on
    it (directly or through other ops); otherwise the two are unordered in the
    launch and the plan is refused.  Two decode layers that reuse the same
    activation buffers (as a decode loop does) are accepted: every reuse is
    reached through the layer-to-layer dependency."""
    h = [_buf(), _buf()]
    l0 = layer_ops(0, h_in=h[0], h_out=h[1])
    l1 = layer_ops(6, h_in=h[1], h_out=h[0])
    # layer 1 reuses layer 0's q/k/v/h1/act buffers
    for i in range(6):
        l1[i]["y"] = l0[i]["y"]
    assert gq.chain_workspace_bytes(gq.FMT_Q4_K, l0 + l1) > 0
    x, y, z = _buf(), _buf(), _buf()
    # write-after-read with no path: op 1 overwrites op 0's input
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, y=y), _op(64, 256, x=z, y=x)])
    # the same with a dependency: accepted
    assert gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, y=y), _op(64, 256, x=y, y=x, deps=[0])]) > 0
    # write-after-write with no path
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, y=y), _op(64, 256, x=z, y=y)])
    # overwriting an earlier op's residual or RMSNorm weight with no path
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, resid=z, y=y), _op(64, 256, x=x, y=z)])
    g = _buf()
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, gamma=g, y=y), _op(64, 256, x=x, y=g)])
    # a transitive path is enough: 2 -> 1 -> 0
    assert gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, y=y), _op(64, 256, x=y, y=z, deps=[0]),
                                                  _op(64, 256, x=z, y=x, deps=[1])]) > 0
    # an op's y aliasing its own input
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, y=x)])
    # partial overlap counts (y of 64 floats starting 32 floats into x)
    with pytest.raises(gq.GQError):
        gq.chain_workspace_bytes(gq.FMT_Q4_K, [_op(64, 256, x=x, y=y), _op(64, 256, x=z, y=_T(x.addr + 128))])

"""The C ABI of libmamba_hip.so, checked on the CPU (no kernel is launched).

- every function include/mamba_hip.h declares is exported by the library;
- the ctypes argument blocks have the library's sizes and field offsets;
- argument checks reject bad calls with the documented codes and messages
  before anything touches a device, and the Python layer maps them to the
  reference's exception types (ValueError / NotImplementedError);
- the Python API refuses CPU tensors instead of falling back to a CPU path.
"""

import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mamba_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mcpu_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for want in ("mcpu_selective_scan_fwd", "mcpu_selective_scan_bwd",
                 "mcpu_selective_scan_bwd_workspace_size", "mcpu_selective_scan_ckpt_size",
                 "mcpu_selective_scan_fwd_workspace_size",
                 "mcpu_causal_conv1d_fwd", "mcpu_causal_conv1d_bwd",
                 "mcpu_causal_conv1d_bwd_workspace_size", "mcpu_causal_conv1d_update",
                 "mcpu_selective_state_update", "mcpu_last_error", "mcpu_version",
                 "mcpu_check_device", "mcpu_args_size"):
        assert want in names


def test_library_exports_every_declared_symbol():
    from mamba_cpu import _C

    missing = [n for n in declared_functions() if not hasattr(_C.lib, n)]
    assert missing == []


def test_library_is_built_for_gfx950():
    from mamba_cpu import _C

    path = _C.LIB_PATH
    assert os.path.exists(path)
    blob = open(path, "rb").read()
    assert b"gfx950" in blob
    assert "gfx950" in _C.version()


def test_argument_blocks_match_the_library():
    from mamba_cpu import _C

    for name, cls in (("scan", _C.ScanArgs), ("conv", _C.ConvArgs),
                      ("conv_update", _C.ConvUpdateArgs), ("state_update", _C.StateUpdateArgs),
                      ("ssd", _C.SsdArgs), ("mixer_step", _C.MixerStepArgs),
                      ("norm_linear", _C.NormLinearArgs), ("mamba2_step", _C.Mamba2StepArgs)):
        assert _C.lib.mcpu_args_size(name.encode()) == ctypes.sizeof(cls)
    assert _C.lib.mcpu_args_size(b"nonsense") == 0


def _header_field_names(struct):
    text = open(HEADER).read()
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        decl = re.sub(r"\[\d+\]", "", decl)
        head, _, rest = decl.rpartition(" ")
        names += [n.strip().lstrip("*") for n in (rest if "," not in decl else
                                                   decl.split(None, 1)[1].replace("*", "")).split(",")]
    return [n for n in names if n]


@pytest.mark.parametrize("struct,cls_name", [("mcpu_scan_args", "ScanArgs"),
                                             ("mcpu_conv_args", "ConvArgs"),
                                             ("mcpu_conv_update_args", "ConvUpdateArgs"),
                                             ("mcpu_state_update_args", "StateUpdateArgs"),
                                             ("mcpu_ssd_args", "SsdArgs"),
                                             ("mcpu_mixer_step_args", "MixerStepArgs"),
                                             ("mcpu_norm_linear_args", "NormLinearArgs"),
                                             ("mcpu_mamba2_step_args", "Mamba2StepArgs")])
def test_argument_block_fields_follow_the_header(struct, cls_name):
    from mamba_cpu import _C

    cls = getattr(_C, cls_name)
    assert [f[0] for f in cls._fields_] == _header_field_names(struct)


def _scan_args(**kw):
    from mamba_cpu import _C

    a = _C.ScanArgs()
    a.u = a.delta = a.A = a.B = a.C = 16  # non-NULL placeholders: never dereferenced
    a.batch, a.dim, a.seqlen, a.dstate, a.ngroups = 2, 8, 32, 16, 1
    a.dtype = _C.MCPU_F32
    a.u_stride[:] = a.delta_stride[:] = (8 * 32, 32, 1)
    a.B_stride[:] = a.C_stride[:] = (32 * 16, 32 * 16, 16, 1)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _rc(fn, *args):
    from mamba_cpu import _C

    rc = fn(*args)
    return rc, _C.lib.mcpu_last_error().decode()


def test_scan_rejects_bad_arguments_before_touching_a_device():
    from mamba_cpu import _C

    L = _C.lib
    assert _rc(L.mcpu_selective_scan_fwd, None, None, 0, None)[0] == _C.MCPU_ERR_INVALID
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(_scan_args(u=None)), None, 0, None)
    assert rc == _C.MCPU_ERR_INVALID and "required" in msg
    # dstate above 64 runs in state slices, up to 4096
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(_scan_args(dstate=4097)), None, 0, None)
    assert rc == _C.MCPU_ERR_UNSUPPORTED and "dstate" in msg
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(_scan_args(ngroups=3)), None, 0, None)
    assert rc == _C.MCPU_ERR_INVALID and "ngroups" in msg
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(_scan_args(dtype=7)), None, 0, None)
    assert rc == _C.MCPU_ERR_INVALID and "dtype" in msg
    a = _scan_args()
    a.u_stride[1] = -1
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(a), None, 0, None)
    assert rc == _C.MCPU_ERR_INVALID and "stride" in msg
    a = _scan_args()
    a.u_stride[1] = 1 << 40  # tile offsets would not fit 32 bits
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(a), None, 0, None)
    assert rc == _C.MCPU_ERR_UNSUPPORTED and "32-bit" in msg
    # backward: required outputs
    rc, msg = _rc(L.mcpu_selective_scan_bwd, ctypes.byref(_scan_args()), None, 0, None)
    assert rc == _C.MCPU_ERR_INVALID and "du" in msg
    # with no steps the per-step tensors may be NULL (torch's empty tensors
    # are): the forward gets past the argument checks (to the device check on
    # a host without a GPU; with one, it has nothing to write)
    empty = _scan_args(u=None, delta=None, B=None, C=None, seqlen=0)
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(empty), None, 0, None)
    assert "required" not in msg


def test_scan_sizes():
    from mamba_cpu import _C

    a = _scan_args(seqlen=33)
    # checkpoints: float32 state at the start of every 16-step block
    assert _C.lib.mcpu_selective_scan_ckpt_size(ctypes.byref(a)) == 4 * 2 * 8 * 3 * 16
    assert _C.lib.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(a)) > 0
    assert _C.lib.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(_scan_args(dstate=0))) == 0
    # forward chunk workspace: none when the rows fill the GPU, some for one long row
    assert _C.lib.mcpu_selective_scan_fwd_workspace_size(ctypes.byref(_scan_args(batch=64, dim=4096))) == 0
    assert _C.lib.mcpu_selective_scan_fwd_workspace_size(
        ctypes.byref(_scan_args(batch=1, dim=64, seqlen=4096))) > 0


def test_complex_scan_sizes_and_limits():
    """complex_a: checkpoints hold (re, im) pairs, the forward uses no
    workspace up to 32 states and above them (32-state slices) one float per
    slice and output element (the call refuses a smaller one), dstate is at
    most 4096, and the imaginary part
    of the last B/C element counts in the 32-bit offset check."""
    from mamba_cpu import _C

    L = _C.lib
    a = _scan_args(seqlen=33, complex_a=1)
    a.B_stride[:] = a.C_stride[:] = (32 * 16 * 2, 32 * 16 * 2, 2, 2 * 33)
    assert L.mcpu_selective_scan_ckpt_size(ctypes.byref(a)) == 2 * 4 * 2 * 8 * 3 * 16
    assert L.mcpu_selective_scan_fwd_workspace_size(
        ctypes.byref(_scan_args(batch=1, dim=64, seqlen=4096, complex_a=1))) == 0
    assert L.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(a)) > \
        L.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(_scan_args(seqlen=33)))
    big = _scan_args(dstate=96, complex_a=1)
    big.out = 16
    assert L.mcpu_selective_scan_fwd_workspace_size(ctypes.byref(big)) == 4 * 3 * 2 * 8 * 32
    assert L.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(_scan_args(dstate=33, complex_a=1))) > 0
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(_scan_args(dstate=4097, complex_a=1)), None, 0, None)
    assert rc == _C.MCPU_ERR_UNSUPPORTED and "dstate" in msg


def test_scan_without_gfx950_reports_the_device():
    """Valid arguments on a machine without a gfx950 device: a device error, no launch."""
    from mamba_cpu import _C

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    rc, msg = _rc(_C.lib.mcpu_selective_scan_fwd, ctypes.byref(_scan_args(out=32)), None, 0, None)
    assert rc in (_C.MCPU_ERR_DEVICE, _C.MCPU_ERR_HIP)
    assert msg


def test_conv_and_state_update_reject_bad_arguments():
    from mamba_cpu import _C

    L = _C.lib
    c = _C.ConvArgs()
    rc, msg = _rc(L.mcpu_causal_conv1d_fwd, ctypes.byref(c), None)
    assert rc != _C.MCPU_OK and msg  # width 0
    # NULL tensors are accepted only where they hold no elements
    c.batch, c.dim, c.seqlen, c.width = 1, 4, 8, 4
    rc, msg = _rc(L.mcpu_causal_conv1d_fwd, ctypes.byref(c), None)
    assert rc == _C.MCPU_ERR_INVALID and "required" in msg
    c.x = c.weight = 16
    rc, msg = _rc(L.mcpu_causal_conv1d_fwd, ctypes.byref(c), None)
    assert rc == _C.MCPU_ERR_INVALID and "out is required" in msg
    c.out = 16
    c.width = (1 << 16) + 1  # widths up to 65536 run (above 16 on the per-element kernels)
    rc, msg = _rc(L.mcpu_causal_conv1d_fwd, ctypes.byref(c), None)
    assert rc in (_C.MCPU_ERR_INVALID, _C.MCPU_ERR_UNSUPPORTED) and "width" in msg
    u = _C.ConvUpdateArgs()
    u.batch, u.dim, u.seqlen, u.width, u.state_len = 2, 8, 1, 4, 3
    rc, msg = _rc(L.mcpu_causal_conv1d_update, ctypes.byref(u), None)
    assert rc == _C.MCPU_ERR_INVALID and "required" in msg
    s = _C.StateUpdateArgs()
    s.batch, s.nheads, s.headdim, s.dstate, s.ngroups = 1, 2, 4, 16, 1
    rc, msg = _rc(L.mcpu_selective_state_update, ctypes.byref(s), None)
    assert rc == _C.MCPU_ERR_INVALID and "required" in msg
    s.state = s.x = s.dt = s.A = s.B = s.C = s.out = 16  # non-NULL placeholders: never dereferenced
    s.batch, s.nheads, s.headdim, s.dstate, s.ngroups = 1, 2, 4, 16, 1
    s.param_strides = 2
    rc, msg = _rc(L.mcpu_selective_state_update, ctypes.byref(s), None)
    assert rc == _C.MCPU_ERR_INVALID and "param_strides" in msg


def test_conv_workspace_depends_only_on_the_shape():
    """The backward's partials workspace is sized from batch, dim, seqlen and
    width alone (host arithmetic, no device): a time-contiguous and a
    channel-contiguous x of one shape need the same bytes, and that covers the
    channel-contiguous path's partials (one per four 8- to 64-step segments)
    as well as the chunked kernels' (up to 16 threads per row)."""
    from mamba_cpu import _C

    L = _C.lib
    for b, d, l, w in ((8, 3072, 2048, 4), (1, 8, 5, 2), (3, 264, 130, 5), (2, 1536, 100000, 4)):
        sizes = []
        for strides in ((d * l, l, 1), (l * d, 1, d)):
            c = _C.ConvArgs()
            c.x = c.weight = 4096
            c.batch, c.dim, c.seqlen, c.width = b, d, l, w
            c.x_stride[:] = strides
            sizes.append(L.mcpu_causal_conv1d_bwd_workspace_size(ctypes.byref(c)))
        assert sizes[0] == sizes[1] > 0
        tiles, ng = b * ((d + 255) // 256), 8
        while ng > 1 and tiles * -(-l // (8 * ng)) < 8192:
            ng //= 2
        gy = -(-(-(-l // (8 * ng))) // 4)
        assert sizes[0] >= 4 * b * max(gy, min(-(-l // 8), 16)) * d * (w + 1)


def test_status_codes_map_to_the_reference_exceptions():
    from mamba_cpu import _C

    with pytest.raises(ValueError):
        _C.check(_C.MCPU_ERR_INVALID, "x")
    with pytest.raises(NotImplementedError):
        _C.check(_C.MCPU_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _C.check(_C.MCPU_ERR_HIP, "x")
    _C.check(_C.MCPU_OK, "x")


def test_public_api_has_no_cpu_fallback():
    import mamba_cpu

    b, d, l, n = 1, 4, 8, 4
    u = torch.randn(b, d, l)
    A = -torch.rand(d, n)
    B = torch.randn(b, n, l)
    with pytest.raises((ValueError, RuntimeError, NotImplementedError)):
        mamba_cpu.selective_scan_fn(u, u, A, B, B)
    with pytest.raises((ValueError, RuntimeError, NotImplementedError)):
        mamba_cpu.causal_conv1d_fn(u, torch.randn(d, 4))
    with pytest.raises((ValueError, RuntimeError, NotImplementedError)):
        mamba_cpu.selective_state_update(torch.zeros(b, d, n), u[..., 0], u[..., 0], A,
                                         B[..., 0], B[..., 0])


def test_public_api_surface():
    """The names the reference exports (src/mamba_cpu/__init__.py)."""
    import mamba_cpu

    for name in ("selective_scan_fn", "causal_conv1d_fn", "causal_conv1d_update",
                 "selective_state_update", "selective_scan_ref", "causal_conv1d_ref"):
        assert callable(getattr(mamba_cpu, name))
    assert hasattr(torch.ops.mamba_cpu, "selective_scan_fwd")
    assert hasattr(torch.ops.mamba_cpu, "selective_scan_bwd")


def test_public_signatures_equal_the_reference():
    """inspect.signature of each public function equals the reference's
    (parameter names, order and defaults), as the reference pins its ops
    against upstream's (tests/test_upstream.py:21-28). The expected text comes
    from the reference's sources, read with `ast` by
    tests/golden/make_signatures.py into tests/golden/signatures.json."""
    import inspect
    import json

    import mamba_cpu

    with open(os.path.join(ROOT, "tests", "golden", "signatures.json")) as f:
        want = json.load(f)
    assert set(want) == {"selective_scan_fn", "causal_conv1d_fn", "causal_conv1d_update",
                         "selective_state_update", "selective_scan_ref", "causal_conv1d_ref"}
    for name, entry in want.items():
        got = str(inspect.signature(getattr(mamba_cpu, name)))
        assert got == entry["signature"], f"{name}: {got} != {entry['signature']} ({entry['source']})"


def test_scan_bwd_waves_is_checked_and_sizes_the_workspace():
    """bwd_waves = 0 lets the library choose; 4, 8 or 12 pin the backward's
    workgroup width (fewer channel blocks, so a smaller dB/dC partial
    workspace, the wider it is); anything else, complex A or dstate > 16 is
    rejected before any device work."""
    from mamba_cpu import _C

    L = _C.lib

    def ws(**kw):
        a = _scan_args(batch=8, dim=1536, seqlen=1024, ckpt=64, **kw)
        a.u_stride[:] = a.delta_stride[:] = (1536 * 1024, 1024, 1)
        a.B_stride[:] = a.C_stride[:] = (1024 * 16, 1024 * 16, 16, 1)
        return L.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(a))

    w4, w8, w12 = ws(bwd_waves=4), ws(bwd_waves=8), ws(bwd_waves=12)
    assert w4 > w8 > w12 > 0
    # the shape of the training-step workload chooses 12 waves by itself
    assert ws() == w12
    for bad in (3, 16, -4):
        rc, msg = _rc(L.mcpu_selective_scan_bwd, ctypes.byref(_scan_args(bwd_waves=bad)), None, 0, None)
        assert rc == _C.MCPU_ERR_INVALID and "bwd_waves" in msg
        assert ws(bwd_waves=bad) == 0
    rc, msg = _rc(L.mcpu_selective_scan_fwd, ctypes.byref(_scan_args(bwd_waves=8, dstate=32)), None, 0, None)
    assert rc == _C.MCPU_ERR_INVALID and "bwd_waves" in msg


def test_conv_update_ring_buffer_needs_a_slot():
    """cache_seqlens with a zero-length conv_state (possible at width 1) would
    index the ring modulo 0: rejected before any device work."""
    from mamba_cpu import _C

    L = _C.lib
    u = _C.ConvUpdateArgs()
    u.x = u.conv_state = u.weight = u.out = u.cache_seqlens = 16
    u.batch, u.dim, u.seqlen, u.width, u.state_len = 1, 4, 1, 1, 0
    rc, msg = _rc(L.mcpu_causal_conv1d_update, ctypes.byref(u), None)
    assert rc == _C.MCPU_ERR_INVALID and "cache_seqlens" in msg


@pytest.mark.gpu
def test_scan_writes_outputs_through_their_strides():
    """out, du, ddelta and dz land at the strides the caller gives: here
    interleaved halves of (batch, seqlen, 2 dim) buffers, as a fused mixer
    writes dz next to the conv's dx. Compared with the contiguous results of
    the same call."""
    from mamba_cpu import _C

    torch.manual_seed(3)
    b, d, l, n = 2, 40, 53, 16
    dev = "cuda"
    u, delta, z, dout = (torch.randn(b, d, l, device=dev) for _ in range(4))
    delta = delta.abs() * 0.1
    A = -torch.rand(d, n, device=dev) - 0.5
    Bk, Ck = torch.randn(b, 1, l, n, device=dev), torch.randn(b, 1, l, n, device=dev)
    D = torch.randn(d, device=dev)

    def args():
        a = _C.ScanArgs()
        a.u, a.delta, a.A, a.B, a.C, a.D, a.z = (t.data_ptr() for t in (u, delta, A, Bk, Ck, D, z))
        a.batch, a.dim, a.seqlen, a.dstate, a.ngroups = b, d, l, n, 1
        a.delta_softplus, a.dtype = 1, _C.MCPU_F32
        a.u_stride[:] = a.delta_stride[:] = a.z_stride[:] = a.dout_stride[:] = u.stride()
        a.B_stride[:], a.C_stride[:] = Bk.stride(), Ck.stride()
        a.dout = dout.data_ptr()
        return a

    stream = torch.cuda.current_stream().cuda_stream

    def call(fwd, a):
        if fwd:
            ws_n = _C.lib.mcpu_selective_scan_fwd_workspace_size(ctypes.byref(a))
        else:
            ws_n = _C.lib.mcpu_selective_scan_bwd_workspace_size(ctypes.byref(a))
        ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device=dev)
        fn = _C.lib.mcpu_selective_scan_fwd if fwd else _C.lib.mcpu_selective_scan_bwd
        rc = fn(ctypes.byref(a), ws.data_ptr(), ws_n, stream)
        assert rc == 0, _C.lib.mcpu_last_error().decode()
        torch.cuda.synchronize()

    small = dict(dA=torch.empty(d, n, device=dev), dB=torch.zeros(b, 1, l, n, device=dev),
                 dC=torch.zeros(b, 1, l, n, device=dev), dD=torch.empty(d, device=dev))
    # Contiguous reference results.
    ref = {k: torch.empty(b, d, l, device=dev) for k in ("out", "du", "ddelta", "dz")}
    a = args()
    a.out = ref["out"].data_ptr()
    call(True, a)
    a = args()
    a.du, a.ddelta, a.dz = ref["du"].data_ptr(), ref["ddelta"].data_ptr(), ref["dz"].data_ptr()
    for k, t in small.items():
        setattr(a, k, t.data_ptr())
    call(False, a)
    # Strided: each output is one half of a (b, l, 2d) buffer, the other half a sentinel.
    bufs = {k: torch.full((b, l, 2 * d), 7.0, device=dev) for k in ref}
    views = {k: bufs[k][..., d:].transpose(1, 2) for k in ref}
    a = args()
    a.out = views["out"].data_ptr()
    a.out_stride[:] = views["out"].stride()
    call(True, a)
    a = args()
    for k, f in (("du", "du"), ("ddelta", "ddelta"), ("dz", "dz")):
        setattr(a, f, views[k].data_ptr())
        getattr(a, f + "_stride")[:] = views[k].stride()
    for k, t in small.items():
        setattr(a, k, t.data_ptr())
    call(False, a)
    for k in ref:
        torch.testing.assert_close(views[k], ref[k], rtol=0, atol=0, msg=lambda m: f"{k}: {m}")
        assert (bufs[k][..., :d] == 7.0).all(), f"{k} wrote outside its view"


@pytest.mark.gpu
@pytest.mark.parametrize("silu", [0, 1])
def test_conv_backward_with_initial_states_but_no_dinitial_states(silu):
    """A C-ABI caller may give initial_states without asking for their
    gradient. With channel-contiguous x (the layout whose fast kernels take no
    initial states) dx, dweight and dbias must still see the initial states in
    the first width-1 taps: checked against the float64 oracle (rtol 1e-4,
    atol 1e-5)."""
    from conftest import assert_close_report
    from mamba_cpu import _C
    from oracle import numerics as O

    torch.manual_seed(5)
    b, d, l, w = 2, 64, 37, 4
    dev = "cuda"
    x = torch.randn(b, l, d, device=dev).transpose(1, 2)          # channel-contiguous view
    dout = torch.randn(b, l, d, device=dev).transpose(1, 2)
    weight, bias = torch.randn(d, w, device=dev), torch.randn(d, device=dev)
    init = torch.randn(b, d, w - 1, device=dev)
    dx = torch.empty(b, l, d, device=dev).transpose(1, 2)
    dweight, dbias = torch.empty(d, w, device=dev), torch.empty(d, device=dev)
    a = _C.ConvArgs()
    a.x, a.weight, a.bias, a.initial_states = x.data_ptr(), weight.data_ptr(), bias.data_ptr(), init.data_ptr()
    a.batch, a.dim, a.seqlen, a.width, a.silu, a.dtype = b, d, l, w, silu, _C.MCPU_F32
    a.x_stride[:], a.init_stride[:] = x.stride(), init.stride()
    a.dout, a.dx, a.dweight, a.dbias = dout.data_ptr(), dx.data_ptr(), dweight.data_ptr(), dbias.data_ptr()
    a.dout_stride[:], a.dx_stride[:] = dout.stride(), dx.stride()
    n = _C.lib.mcpu_causal_conv1d_bwd_workspace_size(ctypes.byref(a))
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
    rc = _C.lib.mcpu_causal_conv1d_bwd(ctypes.byref(a), ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _C.lib.mcpu_last_error().decode()
    torch.cuda.synchronize()
    want = O.causal_conv1d_bwd(x, weight, bias, init, dout, activation="silu" if silu else None)
    for name, got, ref in (("dx", dx, want[0]), ("dweight", dweight, want[1]), ("dbias", dbias, want[2])):
        assert_close_report(got, ref, 1e-4, 1e-5, name)


def _ssd_args(**kw):
    from mamba_cpu import _C

    a = _C.SsdArgs()
    a.x = a.dt = a.A = a.B = a.C = a.out = 16  # non-NULL placeholders: never dereferenced
    a.batch, a.seqlen, a.nheads, a.headdim, a.ngroups, a.dstate = 2, 100, 4, 32, 2, 64
    a.dtype = _C.MCPU_F32
    a.dt_limit_lo, a.dt_limit_hi = 0.0, float("inf")
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_ssd_rejects_bad_arguments_before_touching_a_device():
    from mamba_cpu import _C

    L = _C.lib
    fwd = lambda a: _rc(L.mcpu_ssd_fwd, ctypes.byref(a), None, 0, None)  # noqa: E731
    assert _rc(L.mcpu_ssd_fwd, None, None, 0, None)[0] == _C.MCPU_ERR_INVALID
    for kw, code, word in ((dict(x=None), _C.MCPU_ERR_INVALID, "required"),
                           (dict(headdim=24), _C.MCPU_ERR_UNSUPPORTED, "headdim"),
                           (dict(headdim=80), _C.MCPU_ERR_UNSUPPORTED, "headdim"),
                           (dict(dstate=136), _C.MCPU_ERR_UNSUPPORTED, "dstate"),
                           (dict(ngroups=3), _C.MCPU_ERR_INVALID, "ngroups"),
                           (dict(dtype=7), _C.MCPU_ERR_INVALID, "dtype"),
                           (dict(dt_limit_lo=1.0, dt_limit_hi=0.5), _C.MCPU_ERR_INVALID, "dt_limit"),
                           (dict(head_block=3), _C.MCPU_ERR_INVALID, "head_block"),
                           (dict(head_block=16), _C.MCPU_ERR_INVALID, "head_block"),
                           (dict(chunk_pass=3), _C.MCPU_ERR_INVALID, "chunk_pass"),
                           (dict(chunk_pass=-1), _C.MCPU_ERR_INVALID, "chunk_pass")):
        rc, msg = fwd(_ssd_args(**kw))
        assert rc == code and word in msg, (kw, rc, msg)
    # a saved buffer is needed once there are steps; an empty sequence needs none
    rc, msg = fwd(_ssd_args())
    assert rc == _C.MCPU_ERR_INVALID and "saved" in msg
    rc, msg = _rc(L.mcpu_ssd_bwd, ctypes.byref(_ssd_args()), None, 0, None, 0, None)
    assert rc == _C.MCPU_ERR_INVALID and "dout" in msg
    # tiles move four elements at a time: storage must start on 16 bytes
    rc, msg = fwd(_ssd_args(B=24))
    assert rc == _C.MCPU_ERR_INVALID and "aligned" in msg


def test_ssd_varlen_states_rejects_bad_arguments_before_touching_a_device():
    from mamba_cpu import _C

    L = _C.lib
    var = lambda a, cu=16, n=2, out=16, saved=None, nbytes=0: _rc(  # noqa: E731
        L.mcpu_ssd_varlen_states, ctypes.byref(a), saved, nbytes, cu, n, out, None)
    rc, msg = var(_ssd_args())
    assert rc == _C.MCPU_ERR_INVALID and "batch 1" in msg
    one = _ssd_args(batch=1)
    rc, msg = var(one, n=-1)
    assert rc == _C.MCPU_ERR_INVALID and "count" in msg
    rc, msg = var(one, cu=None)
    assert rc == _C.MCPU_ERR_INVALID and "cu_seqlens" in msg
    rc, msg = var(one, out=None)
    assert rc == _C.MCPU_ERR_INVALID and "varlen_states" in msg
    rc, msg = var(one)
    assert rc == _C.MCPU_ERR_INVALID and "saved" in msg
    rc, msg = var(_ssd_args(batch=1, headdim=24))
    assert rc == _C.MCPU_ERR_UNSUPPORTED and "headdim" in msg
    # no sequences: nothing to do, nothing touched
    assert var(one, cu=None, n=0, out=None)[0] == _C.MCPU_OK


def test_ssd_sizes_follow_the_layout():
    """The saved buffer holds three float32 (batch, nheads, nchunks, 64) arrays
    and the per-chunk states, each 256-byte aligned; the Python fake kernel
    uses the same count; empty inputs need nothing; rejected ones report 0."""
    from mamba_cpu import _C
    from mamba_cpu.ops.ssd_combined import _saved_bytes

    L = _C.lib
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    for b, l, h, p, g, n in ((2, 100, 4, 32, 2, 64), (1, 64, 3, 16, 1, 16), (3, 1, 2, 64, 2, 128)):
        a = _ssd_args(batch=b, seqlen=l, nheads=h, headdim=p, ngroups=g, dstate=n)
        nch = -(-l // 64)
        want = 3 * al(4 * b * h * nch * 64) + al(4 * b * nch * h * p * n)
        assert L.mcpu_ssd_saved_size(ctypes.byref(a)) == want == _saved_bytes(b, l, h, p, n)
        assert L.mcpu_ssd_bwd_workspace_size(ctypes.byref(a)) >= 4 * b * nch * h * p * n
    # dB/dC partials are per head block: pinning 2 heads per block halves them
    one = L.mcpu_ssd_bwd_workspace_size(ctypes.byref(_ssd_args(head_block=1)))
    two = L.mcpu_ssd_bwd_workspace_size(ctypes.byref(_ssd_args(head_block=2)))
    assert one - two == 2 * (al(4 * 2 * 100 * 4 * 64) - al(4 * 2 * 100 * 2 * 64))
    # dL/dcs_last shares per chunk: 8 slices of 256 state elements in the
    # two-launch form, one column block of 64 states in the in-order one
    sep = L.mcpu_ssd_bwd_workspace_size(ctypes.byref(_ssd_args(chunk_pass=1)))
    ino = L.mcpu_ssd_bwd_workspace_size(ctypes.byref(_ssd_args(chunk_pass=2)))
    assert sep - ino == al(4 * 2 * 4 * 2 * 8) - al(4 * 2 * 4 * 2 * 1)
    assert (L.mcpu_ssd_saved_size(ctypes.byref(_ssd_args(chunk_pass=1)))
            == L.mcpu_ssd_saved_size(ctypes.byref(_ssd_args(chunk_pass=2))))
    assert L.mcpu_ssd_saved_size(ctypes.byref(_ssd_args(seqlen=0))) == 0
    assert L.mcpu_ssd_bwd_workspace_size(ctypes.byref(_ssd_args(batch=0))) == 0
    assert L.mcpu_ssd_saved_size(ctypes.byref(_ssd_args(headdim=24))) == 0


def _step_args(**kw):
    from mamba_cpu import _C

    a = _C.MixerStepArgs()
    for f in ("hidden", "in_w", "conv_w", "conv_state", "x_w", "dt_w", "A", "ssm_state", "out_w", "out"):
        setattr(a, f, 256)  # non-NULL placeholders: never dereferenced
    a.batch, a.d_model, a.d_inner, a.dt_rank, a.dstate, a.width, a.state_len = 4, 768, 1536, 48, 16, 4, 4
    a.norm_eps = 1e-5
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_mixer_step_rejects_bad_arguments_before_touching_a_device():
    from mamba_cpu import _C

    L = _C.lib
    step = lambda a, ws=None, n=0: _rc(L.mcpu_mixer_step, ctypes.byref(a), ws, n, None)  # noqa: E731
    assert _rc(L.mcpu_mixer_step, None, None, 0, None)[0] == _C.MCPU_ERR_INVALID
    for kw, code, word in ((dict(hidden=None), _C.MCPU_ERR_INVALID, "required"),
                           (dict(batch=9), _C.MCPU_ERR_UNSUPPORTED, "batch"),
                           (dict(d_model=770), _C.MCPU_ERR_UNSUPPORTED, "multiples of 4"),
                           (dict(state_len=9), _C.MCPU_ERR_UNSUPPORTED, "conv state"),
                           (dict(width=4, state_len=2), _C.MCPU_ERR_UNSUPPORTED, "conv state"),
                           (dict(dstate=256), _C.MCPU_ERR_UNSUPPORTED, "dstate"),
                           (dict(dt_rank=1793, dstate=128), _C.MCPU_ERR_UNSUPPORTED, "dt_rank"),
                           (dict(batch=8, d_inner=8192), _C.MCPU_ERR_UNSUPPORTED, "LDS"),
                           (dict(dtype=5), _C.MCPU_ERR_INVALID, "dtype"),
                           (dict(dtype=_C.MCPU_BF16, hidden_dtype=_C.MCPU_F16), _C.MCPU_ERR_INVALID, "dtype"),
                           (dict(in_w=260), _C.MCPU_ERR_INVALID, "aligned")):
        rc, msg = step(_step_args(**kw))
        assert rc == code and word in msg, (kw, rc, msg)
    rc, msg = step(_step_args())
    assert rc == _C.MCPU_ERR_INVALID and "workspace" in msg


def test_mixer_step_workspace_holds_the_step_vectors():
    """Three (batch, d_inner) float32 vectors (conv outputs, z, gated
    output) plus x_proj's inputs to the state update: at Mamba-130M widths
    the partial x_proj sums of the 192 in_proj workgroups holding x rows
    (8 channels each) for the 80 outputs (dt_rank 48 + 2 x dstate 16), at
    Mamba-2.8B widths (320 such workgroups of 16 channels, 192 outputs: more
    than the state-update workgroup adds at once) the finished x_proj rows."""
    from mamba_cpu import _C

    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    size = lambda **kw: _C.lib.mcpu_mixer_step_workspace_size(ctypes.byref(_step_args(**kw)))  # noqa: E731
    assert size() == 3 * al(4 * 4 * 1536) + al(4 * 4 * 80 * 192)
    assert size(batch=2, d_model=2560, d_inner=5120, dt_rank=160) == 3 * al(2 * 4 * 5120) + al(2 * 4 * 192)
    assert size(batch=9) == 0


def _head_args(**kw):
    from mamba_cpu import _C

    a = _C.NormLinearArgs()
    for f in ("hidden", "weight", "out"):
        setattr(a, f, 256)  # non-NULL placeholders: never dereferenced
    a.batch, a.d_in, a.d_out, a.norm_eps = 4, 768, 50280, 1e-5
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_norm_linear_rejects_bad_arguments_before_touching_a_device():
    from mamba_cpu import _C

    L = _C.lib
    call = lambda a: _rc(L.mcpu_norm_linear, ctypes.byref(a), None)  # noqa: E731
    assert _rc(L.mcpu_norm_linear, None, None)[0] == _C.MCPU_ERR_INVALID
    for kw, code, word in ((dict(weight=None), _C.MCPU_ERR_INVALID, "required"),
                           (dict(batch=0), _C.MCPU_ERR_INVALID, "sizes"),
                           (dict(batch=9), _C.MCPU_ERR_UNSUPPORTED, "batch"),
                           (dict(d_in=770), _C.MCPU_ERR_UNSUPPORTED, "multiple of 4"),
                           (dict(batch=8, d_in=4096), _C.MCPU_ERR_UNSUPPORTED, "LDS"),
                           (dict(dtype=_C.MCPU_BF16, hidden_dtype=_C.MCPU_F16), _C.MCPU_ERR_INVALID, "dtype"),
                           (dict(out_dtype=9), _C.MCPU_ERR_INVALID, "dtype"),
                           (dict(norm_eps=-1.0), _C.MCPU_ERR_INVALID, "norm_eps"),
                           (dict(norm_weight=264), _C.MCPU_ERR_INVALID, "aligned")):
        rc, msg = call(_head_args(**kw))
        assert rc == code and word in msg, (kw, rc, msg)


def _m2_args(**kw):
    from mamba_cpu import _C

    a = _C.Mamba2StepArgs()
    for f in ("hidden", "in_w", "conv_w", "conv_state", "A", "ssm_state", "gate_norm_weight", "out_w", "out"):
        setattr(a, f, 256)  # non-NULL placeholders: never dereferenced
    a.batch, a.d_model, a.d_inner, a.nheads, a.headdim, a.ngroups, a.dstate = 4, 768, 1536, 24, 64, 1, 128
    a.width, a.state_len, a.norm_eps, a.gate_norm_eps = 4, 4, 1e-5, 1e-5
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_mamba2_step_rejects_bad_arguments_before_touching_a_device():
    """Argument checks of mcpu_mamba2_step, and its workspace: the conv
    outputs (x, B, C), the gate and dt rows (padded to a multiple of 4) and
    the scan output, float32 per batch row."""
    from mamba_cpu import _C

    L = _C.lib
    step = lambda a: _rc(L.mcpu_mamba2_step, ctypes.byref(a), None, 0, None)  # noqa: E731
    assert _rc(L.mcpu_mamba2_step, None, None, 0, None)[0] == _C.MCPU_ERR_INVALID
    for kw, code, word in ((dict(gate_norm_weight=None), _C.MCPU_ERR_INVALID, "required"),
                           (dict(d_inner=1500), _C.MCPU_ERR_INVALID, "nheads x headdim"),
                           (dict(ngroups=5), _C.MCPU_ERR_INVALID, "ngroups"),
                           (dict(batch=9), _C.MCPU_ERR_UNSUPPORTED, "batch"),
                           (dict(dstate=256), _C.MCPU_ERR_UNSUPPORTED, "dstate"),
                           (dict(width=9), _C.MCPU_ERR_UNSUPPORTED, "conv width"),
                           (dict(batch=8, d_model=4096), _C.MCPU_ERR_UNSUPPORTED, "LDS"),
                           (dict(dtype=5), _C.MCPU_ERR_INVALID, "dtype"),
                           (dict(out_w=264), _C.MCPU_ERR_INVALID, "aligned")):
        rc, msg = step(_m2_args(**kw))
        assert rc == code and word in msg, (kw, rc, msg)
    al = lambda n: (n + 255) // 256 * 256  # noqa: E731
    want = al(4 * 4 * (1536 + 256)) + al(4 * 4 * 1560) + al(4 * 4 * 1536)
    assert L.mcpu_mamba2_step_workspace_size(ctypes.byref(_m2_args())) == want
    rc, msg = step(_m2_args())
    assert rc == _C.MCPU_ERR_INVALID and "workspace" in msg


def test_fused_step_lds_rule_is_the_librarys():
    """mamba_cpu.decode sends a model to the fused step only where the
    library takes its shape, so that shapes the kernels refuse keep the
    unfused step instead of raising: its LDS rule must accept exactly what
    check_step (Mamba) and check_step2 (Mamba-2) accept. A workspace size of
    0 is the library's refusal. Widths of the Mamba family up to 8192 at
    every batch size up to 8; among them d_inner 4096 at batch 8, exactly
    at the limit, and 5120 (Mamba-2.8B) at batch 5-8, past it."""
    from mamba_cpu import _C

    import mamba_cpu.decode as dec

    L = _C.lib
    seen = set()
    for batch in range(1, 9):
        for dm in (256, 768, 1024, 1536, 2048, 2560, 4096):
            di = 2 * dm
            a = _step_args(batch=batch, d_model=dm, d_inner=di, dt_rank=(dm + 15) // 16)
            takes = L.mcpu_mixer_step_workspace_size(ctypes.byref(a)) > 0
            assert dec._fused_lds_fits(batch, dm, di) == takes, ("mamba", batch, dm)
            seen.add(takes)
            m2 = _m2_args(batch=batch, d_model=dm, d_inner=di, nheads=di // 64, headdim=64)
            takes = L.mcpu_mamba2_step_workspace_size(ctypes.byref(m2)) > 0
            assert dec._fused_lds_fits(batch, dm, di, gated=True) == takes, ("mamba2", batch, dm)
    assert seen == {True, False}
    assert dec._fused_lds_fits(8, 2048, 4096) and not dec._fused_lds_fits(5, 2560, 5120)

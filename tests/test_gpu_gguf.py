"""GGUF ingestion on the device: tensors parsed from a GGUF file, uploaded
through kq_hip_gguf_upload_tensor / _expert_member, then run by the same
kernels, against the CPU oracle on the bytes that were written.

Bars: uploaded bytes identical to the file's payload; dequantization
bit-exact; routing ids exact; matvec, LM head and MoE outputs per element
within 1e-4 absolute or 1e-3 relative of the oracle, or of the
binary64 value where the oracle's own fp32 sums are off by more
(conftest.assert_close, tests/exact.py)."""
import numpy as np
import pytest

from conftest import assert_close

import exact

import kq_hip
import kq_oracle
import kq_synth as S

pytestmark = pytest.mark.gpu

# A layer of the reference model's format pair at reduced size: Q5_K
# gate/up, Q5_1 routed down, named and shaped as its GGUF stores them
# (dims innermost first).
H, E, K, I, V = 512, 32, 4, 256, 3000
SEED = S.W_MOE + 901


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    c = kq_hip.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    w = S.moe_weights(SEED, H, E, I, I, gate_fmt="Q5_K", down_fmt="Q5_1")
    lm = S.quant_matrix("Q8_0", S.stream_key(S.W_LM_HEAD, S.R_WEIGHT, 901), V, H)
    names = {
        "router": ("blk.0.ffn_gate_inp.weight", kq_hip.TYPE_F32, [H, E]),
        "gate": ("blk.0.ffn_gate_exps.weight", kq_hip.TYPE_Q5_K, [H, I, E]),
        "up": ("blk.0.ffn_up_exps.weight", kq_hip.TYPE_Q5_K, [H, I, E]),
        "down": ("blk.0.ffn_down_exps.weight", kq_hip.TYPE_Q5_1, [I, H, E]),
        "shared_gate": ("blk.0.ffn_gate_shexp.weight", kq_hip.TYPE_Q5_K, [H, I]),
        "shared_up": ("blk.0.ffn_up_shexp.weight", kq_hip.TYPE_Q5_K, [H, I]),
        "shared_down": ("blk.0.ffn_down_shexp.weight", kq_hip.TYPE_Q5_1, [I, H]),
        "shared_gate_weight": ("blk.0.ffn_gate_inp_shexp.weight", kq_hip.TYPE_F32, [H]),
    }
    tensors = [(n, t, d, w[role].tobytes()) for role, (n, t, d) in names.items()]
    tensors.append(("output.weight", kq_hip.TYPE_Q8_0, [H, V], lm.tobytes()))
    md = [("general.architecture", S.GGUF_STRING, "qwen35moe"),
          ("qwen35moe.expert_count", S.GGUF_UINT32, E),
          ("qwen35moe.expert_used_count", S.GGUF_UINT32, K)]
    path = tmp_path_factory.mktemp("gguf") / "layer.gguf"
    path.write_bytes(S.gguf_bytes(tensors, md))
    say(f"gguf {path.stat().st_size} bytes, {len(tensors)} tensors")
    g = kq_hip.Gguf(path)
    yield g, w, lm, names
    g.close()


def upload(ctx, g, name):
    t = g.tensor(name)
    n = t.contents.packed_bytes
    buf = ctx.alloc(n)
    g.upload_tensor(ctx, t, buf, n)
    return buf, n


def test_upload_bytes_identical(ctx, model):
    g, w, lm, names = model
    payload = dict({n: w[r] for r, (n, _, _) in names.items()}, **{"output.weight": lm})
    for name, host in payload.items():
        say(f"upload {name}")
        buf, n = upload(ctx, g, name)
        got = ctx.download(buf, np.uint8, n)
        assert np.array_equal(got, host.view(np.uint8).reshape(-1)), name
        buf.close()


@pytest.mark.parametrize("name,type_id", [("blk.0.ffn_gate_exps.weight", kq_hip.TYPE_Q5_K),
                                          ("blk.0.ffn_down_exps.weight", kq_hip.TYPE_Q5_1),
                                          ("output.weight", kq_hip.TYPE_Q8_0),
                                          ("blk.0.ffn_gate_inp.weight", kq_hip.TYPE_F32)])
def test_dequant_from_file_bit_exact(ctx, model, name, type_id):
    g, w, lm, names = model
    buf, n = upload(ctx, g, name)
    t = g.tensor(name).contents
    out = ctx.alloc(t.element_count * 4)
    assert ctx.dequantize(type_id, buf, n, out, t.element_count) == t.element_count
    got = ctx.download(out, np.float32, t.element_count)
    host = np.frombuffer(ctx.download(buf, np.uint8, n).tobytes(), np.uint8)
    want = kq_oracle.dequantize(type_id, host)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    buf.close()
    out.close()


def test_moe_from_file(ctx, model):
    g, w, lm, names = model
    bufs = {role: upload(ctx, g, n)[0] for role, (n, _, _) in names.items()}
    cfg = kq_hip.MoeConfig(H, E, K, I, I)
    T = 3
    x = S.normal_f32(S.stream_key(SEED, S.R_HIDDEN), T * H).reshape(T, H)
    n = cfg.scratch_bytes(T)
    scratch, dx, dout, dids = ctx.alloc(n), ctx.upload(x), ctx.alloc(T * H * 4), ctx.alloc(T * K * 4)
    ctx.moe_execute(cfg, kq_hip.moe_weights(bufs, kq_hip.TYPE_Q5_K, kq_hip.TYPE_Q5_1), dx, T,
                    dout, dids, scratch, n)
    out = ctx.download(dout, np.float32, T * H).reshape(T, H)
    roles = {"router": kq_oracle.F32, "gate": kq_oracle.Q5_K, "up": kq_oracle.Q5_K,
             "down": kq_oracle.Q5_1, "shared_gate": kq_oracle.Q5_K, "shared_up": kq_oracle.Q5_K,
             "shared_down": kq_oracle.Q5_1, "shared_gate_weight": kq_oracle.F32}
    dims = dict(hidden=H, experts=E, top_k=K, inter=I, shared_inter=I)
    ref, tr = kq_oracle.moe_execute(dims, {k: (t, w[k]) for k, t in roles.items()}, x, trace=True)
    assert np.array_equal(ctx.download(dids, np.uint32, T * K).reshape(T, K), tr["selected_ids"])
    assert_close(out, ref, exact=exact.moe(dims, roles, w, x, tr["selected_ids"]))
    for b in list(bufs.values()) + [scratch, dx, dout, dids]:
        b.close()


@pytest.mark.parametrize("expert", [0, 17, E - 1])
def test_expert_member_matvec(ctx, model, expert):
    g, w, lm, names = model
    t = g.tensor("blk.0.ffn_down_exps.weight")
    off, n = kq_hip.gguf_expert_member(t, expert)
    assert n == H * I // 32 * 24 and off == expert * n
    buf = ctx.alloc(n)
    g.upload_expert(ctx, t, expert, buf, n)
    member = w["down"].view(np.uint8).reshape(-1)[off:off + n]
    assert np.array_equal(ctx.download(buf, np.uint8, n), member)
    x = S.normal_f32(S.stream_key(SEED, S.R_X, expert), I)[None, :]
    dx, dy = ctx.upload(x), ctx.alloc(H * 4)
    ctx.matvec(kq_hip.TYPE_Q5_1, buf, H, I, dx, 1, dy)
    assert_close(ctx.download(dy, np.float32, H)[None, :],
                 kq_oracle.matvec(kq_oracle.Q5_1, member, H, I, x),
                 exact=exact.matvec(kq_oracle.Q5_1, member, H, I, x))
    for b in (buf, dx, dy):
        b.close()


def test_lm_head_from_file(ctx, model):
    g, w, lm, names = model
    buf, n = upload(ctx, g, "output.weight")
    h = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, 901), H)[None, :]
    dh, dl, di = ctx.upload(h), ctx.alloc(V * 4), ctx.alloc(4)
    ctx.lm_head(kq_hip.TYPE_Q8_0, buf, V, H, dh, 1, dl, di)
    logits = ctx.download(dl, np.float32, V)[None, :]
    ref = kq_oracle.matvec(kq_oracle.Q8_0, lm, V, H, h)
    assert_close(logits, ref, exact=exact.matvec(kq_oracle.Q8_0, lm, V, H, h))
    assert ctx.download(di, np.uint32, 1)[0] == int(np.argmax(logits[0]))
    for b in (buf, dh, dl, di):
        b.close()


def test_upload_errors(ctx, model, tmp_path):
    g, w, lm, names = model
    t = g.tensor("blk.0.ffn_gate_exps.weight")
    n = t.contents.packed_bytes
    buf = ctx.alloc(n)
    with pytest.raises(kq_hip.KqError) as e:
        g.upload_tensor(ctx, t, buf, n - 1)
    assert e.value.name == "BUFFER_TOO_SMALL"
    with pytest.raises(kq_hip.KqError) as e:
        g.upload_expert(ctx, t, E, buf, n)
    assert e.value.name == "SPAN_OUT_OF_RANGE"
    # a descriptor of another open GGUF
    other = tmp_path / "other.gguf"
    other.write_bytes(S.gguf_bytes([("blk.0.ffn_gate_exps.weight", kq_hip.TYPE_Q8_0, [32],
                                     bytes(34))],
                                   [("general.architecture", S.GGUF_STRING, "x")]))
    with kq_hip.Gguf(other) as o:
        with pytest.raises(kq_hip.KqError) as e:
            g.upload_tensor(ctx, o.tensor("blk.0.ffn_gate_exps.weight"), buf, n)
        assert e.value.name == "TENSOR_OWNERSHIP_MISMATCH"
    buf.close()


def test_upload_spans_windows_and_staging(ctx, tmp_path):
    """A 1.1 GiB tensor: more than one 1 GiB mapped window and many 16 MiB
    staging chunks, the last one partial. Sparse file of zero Q8_0 blocks
    with marker bytes at the window and chunk edges."""
    blocks = (1100 << 20) // 34
    size = blocks * 34
    path = tmp_path / "big.gguf"
    head = S.gguf_bytes([("big", kq_hip.TYPE_Q8_0, [32, blocks], b"")],
                        [("general.architecture", S.GGUF_STRING, "x")])
    marks = [0, (16 << 20) - 1, 16 << 20, (1 << 30) - 1, 1 << 30, (1 << 30) + (16 << 20),
             size - 1]
    with open(path, "wb") as f:
        f.write(head)
        for m in marks:
            f.seek(len(head) + m)
            f.write(bytes([(m * 7 + 3) % 251 + 1]))
        f.truncate(len(head) + size)
    say(f"big upload {size} bytes")
    with kq_hip.Gguf(path) as g:
        t = g.tensor("big")
        assert t.contents.packed_bytes == size
        buf = ctx.alloc(size)
        g.upload_tensor(ctx, t, buf, size)
        for m in marks:
            lo = max(0, m - 2)
            got = ctx.download(buf.ptr + lo, np.uint8, min(size, m + 3) - lo)
            want = np.zeros(got.size, np.uint8)
            for k in marks:
                if lo <= k < lo + got.size:
                    want[k - lo] = (k * 7 + 3) % 251 + 1
            assert np.array_equal(got, want), m
        buf.close()

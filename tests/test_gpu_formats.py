"""The on-disk and wire formats straight from and to HBM (include/pcp_formats.h),
checked against the writers the reference uses (Python struct as in
tools/prepare_rl_dataset.py, numpy tobytes as in tools/convert_weights.py) and
Python's base64 module (the same RFC 4648 standard alphabet as std.base64.standard).
Everything here is byte work: bit-exact."""
import base64
import struct

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from pcp_amd import formats, step
from pcp_amd._lib import PcpError

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def write_prompts(path, prompts):
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(prompts)))
        for p in prompts:
            f.write(struct.pack("<I", len(p)))
            for t in p:
                f.write(struct.pack("<Q", t))


def test_prompts_file_to_packed_batch(tmp_path):
    rng = np.random.default_rng(31)
    prompts = [list(rng.integers(0, 151936, n)) for n in (5, 0, 37, 600, 1)]
    path = tmp_path / "prompts.bin"
    write_prompts(path, prompts)
    tokens, offsets = formats.load_prompts(str(path))
    assert offsets.cpu().tolist() == [0] + list(np.cumsum([len(p) for p in prompts]))
    assert tokens.cpu().tolist() == [int(t) for p in prompts for t in p]
    # straight into the packing of the training step (completions empty here)
    empty = torch.zeros(0, dtype=torch.int64, device=DEV)
    ids, mask = step.pack_rollouts(tokens, offsets, empty, torch.zeros(6, dtype=torch.int64, device=DEV), 8, 512)
    want_ids, want_mask, ok = orc.pack(tokens.cpu().numpy(), offsets.cpu().numpy(), np.zeros(0, np.int64),
                                       np.zeros(6, np.int64), 8, 512)
    assert ok and np.array_equal(ids.cpu().numpy(), want_ids) and np.array_equal(mask.cpu().numpy(), want_mask)


def test_weights_file_round_trip_with_bf16_copy(tmp_path):
    rng = np.random.default_rng(32)
    counts = [896 * 151936 // 64, 3, 4097, 1000003]            # ragged tensors, ~7 MB
    w = rng.standard_normal(sum(counts)).astype(np.float32)
    path = tmp_path / "weights.bin"
    path.write_bytes(w.tobytes() + b"trailing bytes are ignored")
    dev, bf = formats.load_weights(str(path), counts, bf16=True)
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), w.view(np.uint32))
    assert np.array_equal(bf.view(torch.int16).cpu().numpy().view(np.uint16), orc.bf16_from_f32(w))
    out = tmp_path / "saved.bin"
    formats.save_weights(str(out), dev)
    assert out.read_bytes() == w.tobytes()


@pytest.mark.parametrize("n", [0, 1, 2, 3, 4, 47, 48, 49, 95, 96, 97, 767, 768, 769, 100_003, 1 << 20])
def test_base64_encode_decode_against_python(n):
    data = np.random.default_rng(n).integers(0, 256, n).astype(np.uint8)
    d = torch.from_numpy(data).to(DEV)
    enc = formats.b64encode(d)
    assert enc.cpu().numpy().tobytes() == base64.b64encode(data.tobytes())
    dec = formats.b64decode(enc)
    assert dec.cpu().numpy().tobytes() == data.tobytes()


def test_base64_unaligned_buffers():
    data = np.random.default_rng(1).integers(0, 256, 10_001).astype(np.uint8)
    buf = torch.from_numpy(np.concatenate([np.zeros(1, np.uint8), data])).to(DEV)[1:]     # 1-byte offset
    assert buf.dtype == torch.uint8 and buf.data_ptr() % 16 == 1
    enc = formats.b64encode(buf)
    assert enc.cpu().numpy().tobytes() == base64.b64encode(data.tobytes())
    text = torch.from_numpy(np.frombuffer(b"x" + base64.b64encode(data.tobytes()), np.uint8).copy()).to(DEV)[1:]
    assert formats.b64decode(text).cpu().numpy().tobytes() == data.tobytes()


@pytest.mark.parametrize("bad", [b"QQ=A", b"Q===", b"QR==", b"QUJ=", b"QU*D", b"=QUJ", b"QUJD=QUJ", b"QU J"])
def test_base64_rejects_what_std_base64_rejects(bad):
    """Misplaced padding, non-zero leftover bits ("QR==", "QUJ="), characters outside
    the alphabet: std.base64.standard.Decoder returns InvalidPadding / InvalidCharacter."""
    t = torch.from_numpy(np.frombuffer(bad, np.uint8).copy()).to(DEV)
    with pytest.raises(PcpError) as e:
        formats.b64decode(t)
    assert e.value.code == -1


def test_update_weights_payload_full_size():
    """The UPDATE_WEIGHTS payload of Qwen2.5-0.5B's 494,032,768 f32 weights (1.98 GB):
    encoded on the device and decoded back bit for bit; a sample checked against Python."""
    P = 494_032_768
    gen = torch.Generator(device=DEV).manual_seed(3)
    w = torch.randn(P, device=DEV, generator=gen)
    raw = w.view(torch.uint8)
    enc = formats.b64encode(raw)
    assert enc.numel() == (raw.numel() + 2) // 3 * 4
    head = raw[:3 * 100_000].cpu().numpy().tobytes()
    assert enc[:400_000].cpu().numpy().tobytes() == base64.b64encode(head)
    dec = formats.b64decode(enc)
    assert torch.equal(dec, raw)

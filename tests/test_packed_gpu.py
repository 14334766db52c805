"""Packed model files (tools/repack.py:180-257 format) streamed into device memory:
whole files and selected expert slots arrive byte for byte, the Backend's load_file
keeps the rest of a buffer, and errors (missing file, a range past the end of the file
or of the buffer) are reported, not faulted."""
import numpy as np
import pytest

from apex_amd import hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    d = tmp_path_factory.mktemp("packed")
    manifest, slots, routers = synth.write_packed_model(d, seed=5, layers=2, E=16, H=512, I=256)
    return d, manifest, slots


@pytest.mark.parametrize("chunk,nbuf", [(0, 0), (1 << 16, 2), (12345, 3), (1 << 24, 1)])
def test_layer_file_to_device_is_byte_exact(packed, chunk, nbuf):
    d, manifest, slots = packed
    entry = manifest["layers"][1]
    dst = hip.DeviceArray((entry["size"],), np.uint8)
    hip.file_to_device(d / entry["file"], 0, entry["size"], dst, chunk_bytes=chunk, n_buffers=nbuf)
    hip.synchronize()
    assert np.array_equal(dst.numpy(), slots[1].data)


def test_file_range_to_device(packed):
    d, manifest, slots = packed
    raw = (d / "core.bin").read_bytes()
    t = [x for x in manifest["core"]["tensors"] if x["name"] == "layers.0.router.proj.weight"][0]
    dst = hip.DeviceArray((t["nbytes"] + 64,), np.uint8)
    dst.fill_bytes(0xAB)
    hip.file_to_device(d / "core.bin", t["offset"], t["nbytes"], dst, dst_offset=64)
    hip.synchronize()
    got = dst.numpy()
    assert np.all(got[:64] == 0xAB)
    assert got[64:].tobytes() == raw[t["offset"]:t["offset"] + t["nbytes"]]


def test_selected_experts_to_device(packed):
    d, manifest, slots = packed
    entry = manifest["layers"][0]
    stride = entry["stride"]
    used = sum(p["nbytes"] for p in entry["pieces"])
    experts = [7, 0, 15, 3]
    dst = hip.DeviceArray((len(experts) * stride,), np.uint8)
    dst.fill_bytes(0)
    hip.experts_to_device(d / entry["file"], stride, used, experts, dst, stride,
                          chunk_bytes=1 << 15, n_buffers=3)
    hip.synchronize()
    got = dst.numpy().reshape(len(experts), stride)
    for i, e in enumerate(experts):
        assert np.array_equal(got[i, :used], slots[0].data[e * stride:e * stride + used])
        assert np.all(got[i, used:] == 0)


def test_backend_load_file_keeps_the_rest_of_the_buffer(packed):
    d, manifest, slots = packed
    be = hip.Backend(0)
    try:
        n = 1 << 16
        b = be.allocate(3 * n, "core_weights")
        host = be.contents(b, np.uint8)
        host[:] = 0x5A                        # written through contents(): uploaded first
        be.load_file(b, n, d / "layer_00.bin", 2 * n, n)
        got = be.contents(b, np.uint8)
        assert np.all(got[:n] == 0x5A) and np.all(got[2 * n:] == 0x5A)
        assert np.array_equal(got[n:2 * n], slots[0].data[2 * n:3 * n])
        be.release(b)
    finally:
        be.close()


def test_streaming_errors_are_reported(packed, tmp_path):
    d, manifest, slots = packed
    dst = hip.DeviceArray((1024,), np.uint8)
    with pytest.raises(hip.ApexHipError, match="cannot open"):
        hip.file_to_device(tmp_path / "missing.bin", 0, 16, dst)
    size = manifest["layers"][0]["size"]
    with pytest.raises(hip.ApexHipError, match="past the end"):
        hip.file_to_device(d / "layer_00.bin", size - 8, 16, dst)
    be = hip.Backend(0)
    try:
        b = be.allocate(64, "scratch")
        with pytest.raises(hip.ApexHipError, match="past the end of the buffer"):
            be.load_file(b, 32, d / "layer_00.bin", 0, 64)
        be.release(b)
    finally:
        be.close()

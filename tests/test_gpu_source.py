"""The crate's C handle API (c_ffi.rs:35-341) over a safetensors model
directory: open, prewarm, expert_forward (f32 in, bf16-rounded f32 out),
destroy.  The directory is written by the test: an index file mapping tensor
names to two shards, experts in the compressed-tensors form (packed int32 =
the crate's bytes, bf16 or f16 scales), from the oracle's seeded generators;
each result is compared with the oracle's expert_forward on the same bytes.
The error codes that need no GPU are checked in the CPU tests below."""
import json
import os

import numpy as np
import pytest
import torch

from test_gpu_gemm import assert_bf16_close

BF16, F16 = 0, 1


def write_model(path, experts):
    """experts: {(layer, expert): (hidden, inter, group, sdt, flat bytes)}.
    Even layers go to shard 0, odd to shard 1."""
    shards = [{}, {}]
    for (layer, e), (h, i, g, sdt, flat) in experts.items():
        base = f"language_model.model.layers.{layer}.mlp.experts.{e}."
        sdtype = "F16" if sdt == F16 else "BF16"
        off = 0
        for name, rows, cols in (("gate_proj", i, h), ("up_proj", i, h), ("down_proj", h, i)):
            pb, sb = rows * cols // 2, rows * (cols // g) * 2
            shards[layer % 2][base + name + ".weight_packed"] = ("I32", [rows, cols // 8], flat[off:off + pb])
            off += pb
            shards[layer % 2][base + name + ".weight_scale"] = (sdtype, [rows, cols // g], flat[off:off + sb])
            off += sb
    weight_map = {}
    for si, tensors in enumerate(shards):
        fname = f"model-{si + 1:05d}-of-00002.safetensors"
        hdr, data, pos = {"__metadata__": {"format": "pt"}}, [], 0
        for name, (dt, shape, b) in tensors.items():
            hdr[name] = {"dtype": dt, "shape": shape, "data_offsets": [pos, pos + len(b)]}
            data.append(bytes(b))
            pos += len(b)
            weight_map[name] = fname
        hj = json.dumps(hdr).encode()
        with open(os.path.join(path, fname), "wb") as f:
            f.write(len(hj).to_bytes(8, "little"))
            f.write(hj)
            for b in data:
                f.write(b)
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, f)


def make_expert(orc, h, i, g, sdt, seed):
    flat = orc.fill_bytes(seed, 60, orc.expert_bytes(h, i, g))
    offs, sizes = orc.expert_offsets(h, i, g)
    for s_ in (1, 3, 5):
        flat[offs[s_]:offs[s_] + sizes[s_]] = orc.fill_scales(seed, 61 + s_, sizes[s_] // 2, sdt).view(np.uint8)
    return flat


@pytest.mark.gpu
def test_handle_api_matches_oracle(orc, tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import cascadia_amd as cl

    ex = {(0, 0): (512, 256, 32, BF16), (0, 3): (512, 256, 32, BF16), (1, 1): (512, 384, 64, F16),
          (3, 2): (7168, 2048, 32, BF16)}  # the last at the crate's HIDDEN / INTERMEDIATE / G
    data = {k: (*v, make_expert(orc, *v, 7 + 3 * k[0] + k[1])) for k, v in ex.items()}
    write_model(str(tmp_path), data)
    src = cl.ExpertSource(str(tmp_path))
    src.prewarm(0, 3)
    for (layer, e), (h, i, g, sdt, flat) in data.items():
        x = orc.fill_normal_f32(layer * 10 + e, 77, h)
        out = np.empty(h, np.float32)
        src.expert_forward(layer, e, x, out)
        want_bits = orc.cpu_expert_forward(orc.f32_to_bf16(x), 1, flat, h, i, g, sdt).reshape(-1)
        # output is bf16 widened to f32 (c_ffi.rs:336-338)
        assert np.all((out.view(np.uint32) & 0xFFFF) == 0), "not bf16-valued"
        assert_bf16_close((out.view(np.uint32) >> 16).astype(np.uint16), want_bits, f"expert ({layer}, {e})")
        # a second call (expert resident) gives the same bits
        out2 = np.empty(h, np.float32)
        src.expert_forward(layer, e, x, out2)
        assert np.array_equal(out, out2)
    with pytest.raises(cl.CascadiaInt4Error) as ei:
        src.expert_forward(2, 0, np.zeros(512, np.float32), np.zeros(512, np.float32))
    assert ei.value.rc == -2
    with pytest.raises(cl.CascadiaInt4Error) as ei:
        src.prewarm(0, 1)
    assert ei.value.rc == -2
    src.close()


def test_handle_api_error_codes(tmp_path):
    """Codes that need no GPU: null arguments -1, invalid UTF-8 -2, a directory
    without an index -3, a malformed index -3 (c_ffi.rs:35-56)."""
    import ctypes as C

    import cascadia_amd as cl

    L = cl.lib()
    h = C.c_void_p()
    assert L.cascadia_int4_open_source(None, C.byref(h)) == -1
    assert L.cascadia_int4_open_source(str(tmp_path).encode(), None) == -1
    assert L.cascadia_int4_open_source(b"\xff\xfe-not-utf8", C.byref(h)) == -2
    assert L.cascadia_int4_open_source(str(tmp_path / "missing").encode(), C.byref(h)) == -3
    (tmp_path / "model.safetensors.index.json").write_text('{"weight_map": {"a": ')
    assert L.cascadia_int4_open_source(str(tmp_path).encode(), C.byref(h)) == -3
    (tmp_path / "model.safetensors.index.json").write_text('{"metadata": {}}')
    assert L.cascadia_int4_open_source(str(tmp_path).encode(), C.byref(h)) == -3
    # int4_bin manifests: expert_intermediate 0 is refused (ov_moe.rs:452-457),
    # and without it only the K2.6 reader's fixed 7168 hidden is accepted
    # (runner.rs:697-705 over format.rs:63)
    for inter, hidden in ((0, 3072), (0, 7168), (None, 3072)):
        d = tmp_path / f"bin_{inter}_{hidden}"
        d.mkdir()
        write_int4_bin(str(d), hidden, inter, {}, with_inter=inter is not None)
        assert L.cascadia_int4_open_source(str(d).encode(), C.byref(h)) == -3, (inter, hidden)
    assert L.cascadia_int4_prewarm(None, 0, 0) == -1
    assert L.cascadia_int4_expert_forward(None, 0, 0, None, None) == -1
    L.cascadia_int4_destroy_source(None)  # null-safe


def write_int4_bin(path, hidden, inter, experts, with_inter=True):
    """An int4_bin model directory (manifest.rs:21-80, :137-142): manifest.json
    and experts/layer_LL/expert_EEE.bin flat blobs (format.rs:35-47, G 32,
    bf16 scales).  experts: {(layer, expert): flat bytes}."""
    man = {"arch": "test", "num_layers": 4, "dense_layers": [], "num_experts": 8, "top_k": 2,
           "hidden_size": hidden, "num_kv_heads": 1, "qk_head_dim": 1, "v_head_dim": 1,
           "vocab_size": 1, "eos_token_ids": [], "experts_format": "int4_bin"}
    if with_inter:
        man["expert_intermediate"] = inter
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(man, f)
    for (layer, e), flat in experts.items():
        d = os.path.join(path, "experts", f"layer_{layer:02d}")
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, f"expert_{e:03d}.bin"), "wb") as f:
            f.write(bytes(flat))


@pytest.mark.gpu
@pytest.mark.parametrize("hidden,inter,with_inter", [(3072, 1536, True), (7168, 2048, False)])
def test_int4_bin_directory(orc, tmp_path, hidden, inter, with_inter):
    """The runners' int4_bin layout through the handle API: M2 dims from the
    manifest's expert_intermediate, and K2.6 dims from the crate's defaults
    (no expert_intermediate); a missing or truncated file is -2."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import cascadia_amd as cl

    data = {(1, 5): make_expert(orc, hidden, inter, 32, BF16, 31),
            (2, 0): make_expert(orc, hidden, inter, 32, BF16, 32)}
    write_int4_bin(str(tmp_path), hidden, inter, data, with_inter)
    d = os.path.join(str(tmp_path), "experts", "layer_03")
    os.makedirs(d)
    with open(os.path.join(d, "expert_000.bin"), "wb") as f:
        f.write(bytes(data[(1, 5)][:-2]))  # two bytes short
    src = cl.ExpertSource(str(tmp_path))
    for (layer, e), flat in data.items():
        x = orc.fill_normal_f32(layer, e, hidden)
        out = np.empty(hidden, np.float32)
        src.expert_forward(layer, e, x, out)
        want = orc.cpu_expert_forward(orc.f32_to_bf16(x), 1, flat, hidden, inter, 32, BF16).reshape(-1)
        assert_bf16_close((out.view(np.uint32) >> 16).astype(np.uint16), want, f"bin ({layer}, {e})")
    for layer, e in ((1, 6), (3, 0)):
        with pytest.raises(cl.CascadiaInt4Error) as ei:
            src.prewarm(layer, e)
        assert ei.value.rc == -2
    src.close()
    # with a device present the open gets past hipGetDevice, so -3 here is the
    # manifest's: expert_intermediate 0 (ov_moe.rs:452-457), or no
    # expert_intermediate beside a hidden size other than K2.6's 7168
    import ctypes as C
    h = C.c_void_p()
    for bad_inter, bad_hidden in ((0, hidden), (None, 3072)):
        d = os.path.join(str(tmp_path), f"bad_{bad_inter}_{bad_hidden}")
        os.makedirs(d)
        write_int4_bin(d, bad_hidden, bad_inter, {}, with_inter=bad_inter is not None)
        assert cl.lib().cascadia_int4_open_source(d.encode(), C.byref(h)) == -3


@pytest.mark.gpu
def test_expert_cache_lru(orc, tmp_path, monkeypatch):
    """The LRU of runner.rs:142-258: a two-expert cap evicts the least recently
    used (stats count them), an evicted expert reloads with the same result, a
    byte budget of one expert keeps one, and the environment variable sets the
    cap at open."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import cascadia_amd as cl

    h, i, g = 512, 256, 32
    keys = [(0, 0), (0, 1), (1, 0), (1, 1)]
    data = {k: (h, i, g, BF16, make_expert(orc, h, i, g, BF16, 40 + 2 * k[0] + k[1])) for k in keys}
    write_model(str(tmp_path), data)
    x = orc.fill_normal_f32(5, 5, h)

    def run(src, k):
        out = np.empty(h, np.float32)
        src.expert_forward(*k, x, out)
        return out

    src = cl.ExpertSource(str(tmp_path))
    first = {k: run(src, k) for k in keys}
    assert src.cache_stats()[:2] == (4, 0)
    src.set_cache_limits(max_experts=2)  # lowering evicts the two least recently used
    n, ev, b = src.cache_stats()
    assert (n, ev) == (2, 2)
    per = b // 2
    run(src, keys[0])  # evicted: reloads, evicting (1, 0)
    assert src.cache_stats()[:2] == (2, 3)
    run(src, keys[3])  # resident: no eviction
    assert src.cache_stats()[:2] == (2, 3)
    for k in keys:
        assert np.array_equal(run(src, k), first[k]), f"reloaded expert {k} differs"
    src.set_cache_limits(max_experts=0, max_bytes=per + per // 2)
    assert src.cache_stats()[0] == 1
    run(src, keys[1])
    n, _, b = src.cache_stats()
    assert n == 1 and b == per
    src.close()
    monkeypatch.setenv("CASCADIA_INT4_MAX_CACHED_EXPERTS", "1")
    src = cl.ExpertSource(str(tmp_path))
    for k in keys:
        run(src, k)
    assert src.cache_stats()[:2] == (1, 3)
    src.close()


@pytest.mark.gpu
def test_corrupt_shard_headers(orc, tmp_path):
    """Safetensors headers the crate rejects or reads as 0 (safetensors_source.rs
    :85-109): a header length past the file, and negative or fractional data
    offsets (as_u64().unwrap_or(0): the tensor's length comes out wrong) make
    the expert unreadable, -2; nothing is read out of bounds."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import cascadia_amd as cl

    h, i, g = 512, 256, 32
    write_model(str(tmp_path), {(0, 0): (h, i, g, BF16, make_expert(orc, h, i, g, BF16, 9)),
                                (1, 0): (h, i, g, BF16, make_expert(orc, h, i, g, BF16, 10))})
    shard0 = os.path.join(str(tmp_path), "model-00001-of-00002.safetensors")
    raw = bytearray(open(shard0, "rb").read())
    n = int.from_bytes(raw[:8], "little")
    hdr = json.loads(raw[8:8 + n])
    name = "language_model.model.layers.0.mlp.experts.0.gate_proj.weight_scale"
    a, b = hdr[name]["data_offsets"]
    for bad in ([-4, b], [a + 0.5, b], [a, 1e30]):
        hdr[name]["data_offsets"] = bad
        hj = json.dumps(hdr).encode()
        open(shard0, "wb").write(len(hj).to_bytes(8, "little") + hj + raw[8 + n:])
        src = cl.ExpertSource(str(tmp_path))
        with pytest.raises(cl.CascadiaInt4Error) as ei:
            src.prewarm(0, 0)
        assert ei.value.rc == -2, bad
        src.prewarm(1, 0)  # the other shard is intact
        src.close()
    open(shard0, "wb").write((len(raw) * 4).to_bytes(8, "little") + raw[8:])  # length past EOF
    src = cl.ExpertSource(str(tmp_path))
    with pytest.raises(cl.CascadiaInt4Error) as ei:
        src.prewarm(0, 0)
    assert ei.value.rc == -2
    src.close()


@pytest.mark.gpu
def test_expert_prefetch(orc, tmp_path):
    """The prefetcher (runner.rs:282-360): queued experts become resident in
    HBM without a foreground call, counted as loaded; a later expert_forward
    gives the same result as a cold load; an expert already resident is
    skipped, a missing one is processed but not loaded (its error comes on
    first use); a forward issued while its expert is being prefetched waits
    for that load; the LRU limits still apply; close() with requests queued
    returns."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import cascadia_amd as cl

    h, i, g = 1024, 512, 32
    keys = [(0, e) for e in range(6)]
    data = {k: (h, i, g, BF16, make_expert(orc, h, i, g, BF16, 70 + k[1])) for k in keys}
    write_model(str(tmp_path), data)
    x = orc.fill_normal_f32(6, 6, h)

    def run(src, k):
        out = np.empty(h, np.float32)
        src.expert_forward(*k, x, out)
        return out

    cold = cl.ExpertSource(str(tmp_path))
    want = {k: run(cold, k) for k in keys}
    cold.close()

    src = cl.ExpertSource(str(tmp_path))
    for k in keys[:4]:
        src.prefetch(*k)
    src.prefetch(0, 99)  # not in the directory
    src.prefetch_wait()
    sub, drop, proc, loaded = src.prefetch_stats()
    assert (sub, drop, proc, loaded) == (5, 0, 5, 4)
    assert src.cache_stats()[0] == 4
    for k in keys[:4]:
        assert np.array_equal(run(src, k), want[k]), f"prefetched expert {k}"
    assert src.prefetch_stats()[3] == 4 and src.cache_stats()[0] == 4  # no reload
    src.prefetch(*keys[0])  # resident: skipped
    src.prefetch_wait()
    assert src.prefetch_stats()[2:] == (6, 4)
    with pytest.raises(cl.CascadiaInt4Error) as ei:
        src.prewarm(0, 99)
    assert ei.value.rc == -2
    # a forward right behind its prefetch: waits for that load or loads it itself
    src.prefetch(*keys[4])
    assert np.array_equal(run(src, keys[4]), want[keys[4]])
    src.prefetch_wait()
    # limits: two experts at most, prefetches evict like loads do
    src.set_cache_limits(max_experts=2)
    src.prefetch(*keys[5])
    src.prefetch_wait()
    assert src.cache_stats()[0] == 2
    assert np.array_equal(run(src, keys[5]), want[keys[5]])
    for k in keys:
        src.prefetch(*k)
    src.close()  # queued requests dropped, the thread joined

"""The safetensors loader of both hosts (openSafetensors / bf16ToF32 /
f32Scalar, src/loader.js:4-36): e4b.safetensors (Python) and js/loader.js
(Node).  Pinned against the published format's own implementation, the
`safetensors` package (0.8.0 in this image): files written by it are read by
both hosts byte for byte, and files written by write_safetensors load in it;
bf16ToF32 against torch's bfloat16 -> float32 conversion.  CPU only.

torch is imported when a test runs, not when the module is collected: a
pytest session of GPU tests collects this module too, and a second HIP
runtime (torch's) loaded next to the one libe4b.so already uses makes that
runtime's occupancy queries answer 0.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from e4b.safetensors import SafetensorsError, bf16_to_f32, f32_scalar, open_safetensors, write_safetensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "e4b-webgpu_amd", "js")
NODE = shutil.which("node")


def _torch():
    import torch
    return torch


def save_file(*a, **kw):
    from safetensors.torch import save_file as f
    return f(*a, **kw)


def load_file(*a, **kw):
    from safetensors.torch import load_file as f
    return f(*a, **kw)


def _tensors(seed=0):
    torch = _torch()
    g = torch.Generator().manual_seed(seed)
    return {
        "model.layers.0.input_layernorm.weight": torch.randn(64, generator=g).to(torch.bfloat16),
        "model.layers.0.self_attn.q_proj.weight": torch.randint(-128, 127, (8, 16), generator=g, dtype=torch.int8),
        "model.layers.0.self_attn.q_proj.weight_scale": torch.rand(8, generator=g),
        "model.layers.0.layer_scalar": torch.tensor([0.8125]),
        "model.norm.weight": torch.randn(3, 5, generator=g).to(torch.float16),
        "empty": torch.zeros(0, 4),
    }


def _dt(t):
    torch = _torch()
    return {torch.bfloat16: "BF16", torch.int8: "I8", torch.float32: "F32", torch.float16: "F16"}[t.dtype]


def _raw(t):
    return t.contiguous().view(_torch().uint8).numpy().tobytes() if t.numel() else b""


def test_reads_files_written_by_the_safetensors_package(tmp_path):
    ts = _tensors(1)
    p = str(tmp_path / "ref.safetensors")
    save_file(ts, p, metadata={"format": "pt"})
    f = open_safetensors(p)
    assert set(f.index) == set(ts) and "__metadata__" not in f.index
    for name, t in ts.items():
        got = f.fetch(name)
        assert got["dtype"] == _dt(t) and got["shape"] == list(t.shape)
        assert got["buf"].tobytes() == _raw(t), name
        assert f.has(name) and f.info(name)["data_offsets"] == got["data_offsets"]
    assert not f.has("missing")
    with pytest.raises(SafetensorsError):
        f.fetch("missing")
    w = f.fetch("model.layers.0.input_layernorm.weight")["buf"]
    np.testing.assert_array_equal(bf16_to_f32(w), ts["model.layers.0.input_layernorm.weight"].float().numpy())
    assert f32_scalar(f.fetch("model.layers.0.layer_scalar")["buf"]) == 0.8125
    assert f32_scalar(b"") == 0.0


def test_written_files_load_in_the_safetensors_package(tmp_path):
    ts = _tensors(2)
    p = str(tmp_path / "ours.safetensors")
    write_safetensors(p, {n: (_dt(t), list(t.shape), _raw(t)) for n, t in ts.items()}, {"k": "v"})
    back = load_file(p)
    for name, t in ts.items():
        assert back[name].dtype == t.dtype and _torch().equal(back[name], t), name


def test_bf16_widening_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = bf16_to_f32(bits)
    torch = _torch()
    want = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    np.testing.assert_array_equal(got.view(np.uint32), bits.astype(np.uint32) << 16)


def test_rejects_truncated_and_inconsistent_files(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(b"\x00\x01")
    with pytest.raises(SafetensorsError):
        open_safetensors(str(p))
    h = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}).encode()
    p.write_bytes(len(h).to_bytes(8, "little") + h + b"\x00" * 12)
    with pytest.raises(SafetensorsError):
        open_safetensors(str(p))


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_js_loader_matches_python(tmp_path):
    ts = _tensors(3)
    p = str(tmp_path / "js.safetensors")
    save_file(ts, p, metadata={"format": "pt"})
    script = f"""
const {{ openSafetensors, bf16ToF32, f32Scalar }} = require({json.dumps(os.path.join(JS, 'loader.js'))});
(async () => {{
  const st = openSafetensors({json.dumps(p)});
  const out = {{ index: st.index, bytes: {{}} }};
  for (const n of Object.keys(st.index)) {{
    const t = await st.fetch(n);
    out.bytes[n] = Array.from(new Uint8Array(t.buf));
  }}
  const w = await st.fetch("model.layers.0.input_layernorm.weight");
  out.bf16 = Array.from(new Uint32Array(bf16ToF32(w.buf).buffer));
  out.scalar = f32Scalar((await st.fetch("model.layers.0.layer_scalar")).buf);
  out.has = [st.has("model.norm.weight"), st.has("nope")];
  try {{ await st.fetch("nope"); out.missing = "no error"; }} catch (e) {{ out.missing = e.message; }}
  st.close();
  console.log(JSON.stringify(out));
}})().catch((e) => {{ console.error(e); process.exit(1); }});
"""
    r = subprocess.run([NODE, "-e", script], check=True, capture_output=True, text=True, timeout=60)
    js = json.loads(r.stdout)
    f = open_safetensors(p)
    assert js["index"] == f.index
    for n in ts:
        assert bytes(js["bytes"][n]) == f.fetch(n)["buf"].tobytes(), n
    want = bf16_to_f32(f.fetch("model.layers.0.input_layernorm.weight")["buf"]).view(np.uint32)
    assert js["bf16"] == want.tolist()
    assert js["scalar"] == 0.8125 and js["has"] == [True, False] and "not found" in js["missing"]

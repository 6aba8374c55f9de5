"""Seeded random-init ``evo2-runtime-v1`` Safetensors artifacts.

The file layout and typed metadata follow evo.cpp's artifact profile
(`docs/model-format.md`, reader `src/model_format.cpp:749-1223`, tensor set
and shapes `src/cpu/model.cpp:2651-2874`): an 8-byte little-endian header
length, a JSON header padded with spaces to 8 bytes, then a dense payload in
declaration order with no holes. Metadata values carry the profile's type
prefixes (`s:`, `u:`, `f:` = IEEE-754 f64 bits as 16 lowercase hex digits,
`b:`, `l:`).

Two initialisation profiles are provided:

* ``"survey"`` -- the distributions of the benchmark configurations: linear
  weights N(0, 0.02) rounded to BF16, norm scales 1 + N(0, 0.02), short/HCS/HCM
  taps and D N(0, 0.02), log-poles log U[0.5, 0.99], residues N(0, 0.02).
* ``"unit"`` -- variances chosen so every sub-block contributes O(1) values to
  the residual stream. Parity tests use it so that a wrong Hyena or attention
  kernel visibly moves the logits.
"""
from __future__ import annotations

import json
import math
import struct
from dataclasses import dataclass, field
from typing import Callable, Dict, Iterable, List, Optional, Sequence

import numpy as np

from .fp8 import e4m3_encode

ARCHITECTURE = "StripedHyena2"
PROFILE = "evo2-runtime-v1"
RUNTIME_ABI = "evo2-safetensors-v1"


@dataclass
class ModelShape:
    """StripedHyena2 hyper-parameters (names follow the artifact metadata)."""

    width: int
    layers: int
    heads: int
    inner: int
    hcs: List[int]
    hcm: List[int]
    hcl: List[int]
    attn: List[int]
    vocab: int = 512
    state: int = 16
    short_len: int = 3
    hcs_len: int = 7
    hcm_len: int = 128
    hcs_groups: int = 256
    hcm_groups: int = 256
    max_seqlen: int = 1048576
    eps: float = 1e-6
    rope_base: float = 10000.0
    rope_scale: float = 1.0
    column_split: bool = True
    model_id: str = "random-init"

    @property
    def head_dim(self) -> int:
        return self.width // self.heads

    def mixer(self, index: int) -> str:
        if index in self.attn:
            return "attn"
        if index in self.hcm:
            return "hcm"
        if index in self.hcl:
            return "hcl"
        return "hcs"

    def validate(self) -> None:
        every = sorted(self.hcs + self.hcm + self.hcl + self.attn)
        if every != list(range(self.layers)):
            raise ValueError("mixer lists must cover every block exactly once")
        if self.width % self.heads or self.head_dim % 2:
            raise ValueError("width must split into an even head dimension")
        if self.width % self.hcs_groups or self.width % self.hcm_groups:
            raise ValueError("filter groups must divide the width")


def _pattern(layers: int, attn: Sequence[int]):
    """Evo 2's striping: hcs, hcm, hcl repeating between attention blocks
    (src/model_registry.cpp:56-65)."""
    hcs, hcm, hcl = [], [], []
    kinds = (hcs, hcm, hcl)
    position = 0
    for index in range(layers):
        if index in attn:
            continue
        kinds[position % 3].append(index)
        position += 1
    return hcs, hcm, hcl


def evo2_7b_shape() -> ModelShape:
    """Evo 2 7B topology (`evo2_7b`, src/model_registry.cpp:61-65)."""
    attn = [3, 10, 17, 24, 31]
    hcs, hcm, hcl = _pattern(32, attn)
    return ModelShape(width=4096, layers=32, heads=32, inner=11264, hcs=hcs,
                      hcm=hcm, hcl=hcl, attn=attn, hcs_groups=256,
                      hcm_groups=256, rope_scale=128.0, max_seqlen=1048576,
                      model_id="random-init-evo2-7b-shape")


def evo2_1b_shape() -> ModelShape:
    """Evo 2 1B topology (`evo2_1b_base`, src/model_registry.cpp:56-60)."""
    attn = [3, 10, 17, 24]
    hcs, hcm, hcl = _pattern(25, attn)
    return ModelShape(width=1920, layers=25, heads=15, inner=5120, hcs=hcs,
                      hcm=hcm, hcl=hcl, attn=attn, hcs_groups=128,
                      hcm_groups=128, rope_scale=1.0, max_seqlen=8192,
                      model_id="random-init-evo2-1b-shape")


def tiny_shape(width: int = 64, layers: int = 8, heads: int = 4,
               inner: int = 96, groups: int = 16, attn: Sequence[int] = (3,),
               hcm_len: int = 128, **kwargs) -> ModelShape:
    hcs, hcm, hcl = _pattern(layers, attn)
    return ModelShape(width=width, layers=layers, heads=heads, inner=inner,
                      hcs=hcs, hcm=hcm, hcl=hcl, attn=list(attn),
                      hcs_groups=groups, hcm_groups=groups, hcm_len=hcm_len,
                      model_id=kwargs.pop("model_id", "random-init-tiny"),
                      **kwargs)


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """Round F32 to BF16 (round to nearest even) and return the raw bits."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    rounding = np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))
    return ((bits + rounding) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def _meta_f64(value: float) -> str:
    return "f:" + struct.pack(">d", float(value)).hex()


@dataclass
class TensorSpec:
    name: str
    dtype: str
    shape: List[int]
    make: Callable[[np.random.Generator], np.ndarray]

    @property
    def nbytes(self) -> int:
        width = {"F32": 4, "BF16": 2, "F8_E4M3": 1}[self.dtype]
        return int(np.prod(self.shape)) * width


@dataclass
class Artifact:
    """A seeded artifact description. Tensor i is drawn from its own PCG64
    stream seeded with (seed, i), so the bytes depend only on (shape, seed,
    init, fp8 layers); ``write`` streams them to disk one tensor at a time."""

    shape: ModelShape
    seed: int
    specs: List[TensorSpec] = field(default_factory=list)

    def add(self, name: str, dtype: str, shape: Sequence[int],
            make: Callable[[np.random.Generator], np.ndarray]) -> None:
        self.specs.append(TensorSpec(name, dtype, [int(d) for d in shape], make))

    def _make(self, index: int) -> np.ndarray:
        spec = self.specs[index]
        rng = np.random.Generator(np.random.PCG64(
            np.random.SeedSequence([self.seed, index])))
        array = np.ascontiguousarray(spec.make(rng))
        if list(array.shape) != spec.shape or array.nbytes != spec.nbytes:
            raise AssertionError(f"generator mismatch for {spec.name}")
        return array

    def _stream(self, workers: int = 8):
        """Yield (spec, array) in order; tensors are generated ahead on a
        thread pool (each has its own PCG64 stream, so order and thread count
        do not change the bytes)."""
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=workers) as pool:
            pending = {}
            for index in range(min(workers, len(self.specs))):
                pending[index] = pool.submit(self._make, index)
            for index, spec in enumerate(self.specs):
                array = pending.pop(index).result()
                ahead = index + workers
                if ahead < len(self.specs):
                    pending[ahead] = pool.submit(self._make, ahead)
                yield spec, array

    def tensors(self) -> Dict[str, np.ndarray]:
        """Materialise every tensor (small models only)."""
        return {spec.name: array for spec, array in self._stream()}

    def metadata(self) -> Dict[str, str]:
        s = self.shape
        return {
            "evo2.profile": "s:" + PROFILE,
            "runtime.abi": "s:" + RUNTIME_ABI,
            "model.architecture": "s:" + ARCHITECTURE,
            "model.id": "s:" + s.model_id,
            "config.vocab_size": f"u:{s.vocab}",
            "config.hidden_size": f"u:{s.width}",
            "config.num_layers": f"u:{s.layers}",
            "config.num_attention_heads": f"u:{s.heads}",
            "config.state_size": f"u:{s.state}",
            "config.inner_mlp_size": f"u:{s.inner}",
            "config.short_filter_length": f"u:{s.short_len}",
            "config.hcs_filter_length": f"u:{s.hcs_len}",
            "config.hcm_filter_length": f"u:{s.hcm_len}",
            "config.hcs_filter_groups": f"u:{s.hcs_groups}",
            "config.hcm_filter_groups": f"u:{s.hcm_groups}",
            "config.max_seqlen": f"u:{s.max_seqlen}",
            "config.eps": _meta_f64(s.eps),
            "config.rotary_emb_base": _meta_f64(s.rope_base),
            "config.rotary_emb_scaling_factor": _meta_f64(s.rope_scale),
            "config.column_split": "b:1" if s.column_split else "b:0",
            "config.hcs_layer_idxs": "l:" + ",".join(map(str, s.hcs)),
            "config.hcm_layer_idxs": "l:" + ",".join(map(str, s.hcm)),
            "config.hcl_layer_idxs": "l:" + ",".join(map(str, s.hcl)),
            "config.attn_layer_idxs": "l:" + ",".join(map(str, s.attn)),
        }

    def write(self, path: str) -> None:
        header: Dict[str, object] = {"__metadata__": self.metadata()}
        offset = 0
        for spec in self.specs:
            header[spec.name] = {"dtype": spec.dtype, "shape": spec.shape,
                                 "data_offsets": [offset, offset + spec.nbytes]}
            offset += spec.nbytes
        text = json.dumps(header, separators=(",", ":")).encode()
        text += b" " * ((8 - len(text) % 8) % 8)
        with open(path, "wb") as handle:
            handle.write(struct.pack("<Q", len(text)))
            handle.write(text)
            for _, array in self._stream():
                handle.write(memoryview(array).cast("B"))


def random_artifact(shape: ModelShape, seed: int = 0, init: str = "unit",
                    fp8_layers: Optional[Iterable[int]] = None,
                    fp8_input_amax: float = 8.0) -> Artifact:
    """Describe a seeded random-init artifact.

    ``fp8_layers`` lists Hyena blocks whose input projection is stored as
    software E4M3 codes with ``fp8_runtime_scales = [input_scale,
    output_scale]``: weight_scale = 448 / amax(W), input_scale = 448 /
    fp8_input_amax, output_scale = 1 / (input_scale * weight_scale)
    (the converter's rule `tools/evo/checkpoint.py:393-396`).
    """
    shape.validate()
    if init not in ("unit", "survey"):
        raise ValueError("init must be 'unit' or 'survey'")
    fp8 = set(fp8_layers or ())
    w, f, hd = shape.width, shape.inner, shape.head_dim
    unit = init == "unit"

    def normal(dims, std):
        return lambda rng: (rng.standard_normal(dims, dtype=np.float32)
                            * np.float32(std))

    def bf16(maker):
        return lambda rng: bf16_bits(maker(rng))

    def linear(rows, cols):
        return bf16(normal((rows, cols), 1.0 / math.sqrt(cols) if unit else 0.02))

    def scale_vector(rng):
        return np.float32(1.0) + normal((w,), 0.02)(rng)

    inv_freq = (1.0 / (shape.rope_base ** (np.arange(0, hd, 2, dtype=np.float64)
                                            / hd))).astype(np.float32)
    art = Artifact(shape, seed)
    art.add("embedding_layer.weight", "BF16", (shape.vocab, w),
            bf16(normal((shape.vocab, w), 1.0 if unit else 0.02)))
    art.add("norm.scale", "F32", (w,), scale_vector)
    for index in range(shape.layers):
        p = f"blocks.{index}"
        kind = shape.mixer(index)
        art.add(p + ".pre_norm.scale", "F32", (w,), scale_vector)
        art.add(p + ".post_norm.scale", "F32", (w,), scale_vector)
        if kind == "attn":
            art.add(p + ".inner_mha_cls.Wqkv.weight", "BF16", (3 * w, w),
                    linear(3 * w, w))
            art.add(p + ".inner_mha_cls.out_proj.weight", "BF16", (w, w),
                    linear(w, w))
            art.add(p + ".inner_mha_cls.out_proj.bias", "BF16", (w,),
                    bf16(normal((w,), 0.02)))
            art.add(p + ".inner_mha_cls.rotary_emb.inv_freq", "F32", (hd // 2,),
                    lambda rng: inv_freq.copy())
        else:
            if index in fp8:
                # the codes and their scale tensor are derived from the same
                # weight draw (seeded by the codes tensor's position)
                weight_maker = normal((3 * w, w), 1.0 / math.sqrt(w) if unit else 0.02)
                position = len(art.specs)

                def weight_and_scale(art=art, position=position, maker=weight_maker):
                    rng = np.random.Generator(np.random.PCG64(
                        np.random.SeedSequence([art.seed, position])))
                    weight = maker(rng)
                    return weight, np.float32(448.0) / np.float32(np.abs(weight).max())

                def codes(rng, draw=weight_and_scale):
                    weight, weight_scale = draw()
                    return e4m3_encode(weight * weight_scale)

                def scales(rng, draw=weight_and_scale):
                    _, weight_scale = draw()
                    input_scale = np.float32(448.0) / np.float32(fp8_input_amax)
                    return np.array([input_scale, np.float32(1.0) /
                                     (input_scale * weight_scale)], dtype=np.float32)

                art.add(p + ".projections.weight", "F8_E4M3", (3 * w, w), codes)
                art.add(p + ".projections.fp8_runtime_scales", "F32", (2,), scales)
            else:
                art.add(p + ".projections.weight", "BF16", (3 * w, w),
                        linear(3 * w, w))
            art.add(p + ".filter.short_filter_weight", "BF16",
                    (3 * w, 1, shape.short_len),
                    bf16(normal((3 * w, 1, shape.short_len), 0.5 if unit else 0.02)))
            if kind == "hcs":
                art.add(p + ".filter.h", "BF16", (shape.hcs_groups, 1, shape.hcs_len),
                        bf16(normal((shape.hcs_groups, 1, shape.hcs_len),
                                    0.4 if unit else 0.02)))
            elif kind == "hcm":
                art.add(p + ".filter.D", "BF16", (w,),
                        bf16(normal((w,), 0.5 if unit else 0.02)))
                art.add(p + ".filter.h", "BF16", (shape.hcm_groups, 1, shape.hcm_len),
                        bf16(normal((shape.hcm_groups, 1, shape.hcm_len),
                                    1.0 / math.sqrt(shape.hcm_len) if unit else 0.02)))
            else:
                art.add(p + ".filter.D", "BF16", (w,),
                        bf16(normal((w,), 0.5 if unit else 0.02)))
                art.add(p + ".filter.log_poles", "F32", (w, shape.state, 1),
                        lambda rng: np.log(rng.uniform(0.5, 0.99, size=(
                            w, shape.state, 1))).astype(np.float32))
                art.add(p + ".filter.residues", "F32", (w, shape.state),
                        normal((w, shape.state), 0.1 if unit else 0.02))
            art.add(p + ".out_filter_dense.weight", "BF16", (w, w), linear(w, w))
            art.add(p + ".out_filter_dense.bias", "BF16", (w,),
                    bf16(normal((w,), 0.02)))
        art.add(p + ".mlp.l1.weight", "BF16", (f, w), linear(f, w))
        art.add(p + ".mlp.l2.weight", "BF16", (f, w), linear(f, w))
        art.add(p + ".mlp.l3.weight", "BF16", (w, f), linear(w, f))
    return art


def acgt_tokens(count: int, seed: int = 0) -> np.ndarray:
    """Uniform draws from the ASCII bytes A, C, G, T (byte-identity tokens)."""
    rng = np.random.Generator(np.random.PCG64(seed + 0x5eed))
    return np.frombuffer(b"ACGT", dtype=np.uint8)[
        rng.integers(0, 4, size=count)].astype(np.uint32)

"""The NCA cell as a parameter container whose compute runs in libnca_hip.so.

`NCAConfig` and `NCA` keep the reference's names and parameter layout (reference
src/nca/model.py:47-137 and 304-355): `perceive.weight (K, 1, 3, 3)`, `update.fc1` /
`update.fc2` 1x1 convolutions, `head` (mlp head), and the buffers `embed`, `out_embed`,
`pad_vec`. A reference checkpoint's `model` state dict therefore loads as is
(`NCA(NCAConfig.from_dict(ckpt["model_config"])).load_state_dict(ckpt["model"])`).

Supported cells (what the HIP kernels implement): `perception="kernels"` with 4 kernels, ReLU
MLP, no group normalisation, no time / task embedding, head "mlp" or "l2"; C / hidden of
16 / 128, 32 / 256 or 64 / 256. Other configurations raise ValueError when a HIP operator is
called, like the reference engine rejects option combinations it does not implement
(reference src/nca/engine/step.py:93-105).
"""

from __future__ import annotations

import ctypes
from dataclasses import asdict, dataclass, field

import numpy as np
import torch
from torch import nn

from . import _lib

# 3x3 Moore neighbourhood offsets (dy, dx), row-major, centre included (model.py:43-44)
OFFSETS = [(dy, dx) for dy in (-1, 0, 1) for dx in (-1, 0, 1)]


# Readout coordinates of the maze tokens for the "semantic" embedding, keyed by (vocabulary
# size, c_out): the reference's table (src/nca/embeddings.py:25-28), needed as is so that its
# trained maze cells read the same inputs.
_SEMANTIC_READOUT = {
    (4, 2): ((0.0, -1.0), (0.0, 1.0), (1.0, 0.0), (-1.0, 0.0)),
    (5, 3): ((0.0, 0.0, 0.0), (0.0, 0.0, 1.0), (1.0, 0.0, -1.0), (0.0, -1.0, 1.0), (0.0, 1.0, 1.0)),
}


def make_embeddings(vocab_size: int, dim: int, kind: str = "onehot", seed: int = 0,
                    c_out: int | None = None) -> torch.Tensor:
    """Fixed token embeddings, a (vocab_size, dim) float tensor whose row v is what a given cell
    of token v is clamped to (reference src/nca/embeddings.py:31-53).

    * "onehot": row v is the v-th unit vector (needs dim >= vocab_size);
    * "onehot_inputs": unit vectors for the first min(vocab_size, dim) tokens, zero rows for
      the rest (the maze cells' output-only PATH token is never an input);
    * "semantic": every entry -1 except the first c_out, which hold the token's readout
      coordinates;
    * "orthonormal": the first vocab_size rows of the Q factor of a (dim, dim) standard normal
      matrix drawn from numpy's default_rng(seed).
    """
    if kind == "onehot_inputs":
        return torch.eye(vocab_size, dim)
    if vocab_size > dim:
        raise ValueError(f"{vocab_size} tokens do not fit {dim} embedding channels")
    if kind == "onehot":
        return torch.eye(vocab_size, dim)
    if kind == "semantic":
        coords = _SEMANTIC_READOUT.get((vocab_size, c_out))
        if coords is None:
            raise ValueError(f"no semantic readout coordinates for {vocab_size} tokens and "
                             f"c_out={c_out}")
        e = -torch.ones(vocab_size, dim)
        e[:, :c_out] = torch.tensor(coords)
        return e
    if kind == "orthonormal":
        gauss = np.random.default_rng(seed).standard_normal((dim, dim))
        basis = np.linalg.qr(gauss)[0]
        return torch.from_numpy(np.ascontiguousarray(basis[:vocab_size])).to(torch.float32)
    raise ValueError(f"embedding kind {kind!r} (onehot | onehot_inputs | semantic | orthonormal)")


def fixed_kernels() -> torch.Tensor:
    """Identity, Sobel-x / 8, Sobel-y / 8 (reference model.py:199-201: cross-correlation,
    sy = sx.T) and the Laplacian [[1, 2, 1], [2, -12, 2], [1, 2, 1]] / 16 of Mordvintsev et al.'s
    texture NCA. (4, 1, 3, 3)."""
    ident = torch.tensor([[0.0, 0, 0], [0, 1, 0], [0, 0, 0]])
    sx = torch.tensor([[-1.0, 0, 1], [-2, 0, 2], [-1, 0, 1]]) / 8
    lap = torch.tensor([[1.0, 2, 1], [2, -12, 2], [1, 2, 1]]) / 16
    return torch.stack([ident, sx, sx.T, lap])[:, None]


@dataclass
class NCAConfig:
    """Architecture hyper-parameters, same fields as the reference's NCAConfig."""

    vocab_size: int
    channels: int
    c_in: int
    c_out: int
    output_tokens: tuple[int, ...]
    in_offset: int = 0
    out_offset: int = 0
    c_task: int = 0
    n_tasks: int = 0
    embedding: str = "onehot"
    perception: str = "kernels"
    heads: int = 4
    grid_size: tuple[int, int] | None = None
    padding: str = "wall"
    wall_token: int | None = 2
    update: str = "mlp"
    expansion: int = 2
    hidden_from_perception: bool = False
    norm_groups: int = 0
    norm_fired_only: bool = False
    sigma_init: float = 0.15
    init_uniform: bool = False
    fire_rate: float = 0.8
    head: str = "l2"
    time_steps: int = 0
    zero_init_update: bool = True
    attn_bias: bool = True
    project_update: bool = False
    noise_after_norm: bool = False
    norm_init: bool = False
    norm_style: str = "sqrt_eps"
    init_style: str = "torch"
    # build-specific: "fixed" initialises the kernels to identity / Sobel / Sobel / Laplacian
    kernel_init: str = "random"

    def __post_init__(self) -> None:
        self.output_tokens = tuple(int(t) for t in self.output_tokens)
        if self.grid_size is not None:
            self.grid_size = tuple(int(s) for s in self.grid_size)
        c = self.channels
        assert self.in_offset + self.c_in <= c, "input slice exceeds the state"
        assert self.out_offset + self.c_out <= c, "output slice exceeds the state"
        if self.head in ("l2", "cosine"):
            assert self.in_offset <= self.out_offset, "output slice must lie inside the input slice"
            assert self.out_offset + self.c_out <= self.in_offset + self.c_in, (
                "output slice must lie inside the input slice for embedding-based heads"
            )

    @property
    def in_slice(self) -> slice:
        return slice(self.in_offset, self.in_offset + self.c_in)

    @property
    def out_slice(self) -> slice:
        return slice(self.out_offset, self.out_offset + self.c_out)

    @property
    def hidden(self) -> int:
        base = self.heads * self.channels if self.hidden_from_perception else self.channels
        return self.expansion * base

    def to_dict(self) -> dict:
        return asdict(self)

    @classmethod
    def from_dict(cls, d: dict) -> NCAConfig:
        return cls(**d)


class KernelPerception(nn.Module):
    """K shared 3x3 kernels (reference model.py:161-178); the compute is in the HIP kernels."""

    def __init__(self, channels: int, heads: int, init: str = "random"):
        super().__init__()
        w = fixed_kernels() if init == "fixed" else torch.randn(heads, 1, 3, 3) / 3
        if init == "fixed" and heads != 4:
            raise ValueError("fixed kernels need heads=4")
        self.weight = nn.Parameter(w)
        self.channels, self.heads, self.out_dim = channels, heads, heads * channels


class MLPUpdate(nn.Module):
    """fc1 (1x1) -> ReLU -> fc2 (1x1) (reference model.py:277-287)."""

    def __init__(self, in_dim: int, channels: int, hidden: int, zero_init: bool):
        super().__init__()
        self.fc1 = nn.Conv2d(in_dim, hidden, 1)
        self.fc2 = nn.Conv2d(hidden, channels, 1)
        if zero_init:
            nn.init.zeros_(self.fc2.weight)
            nn.init.zeros_(self.fc2.bias)


@dataclass
class _Packed:
    key: tuple
    buf: torch.Tensor
    desc: _lib.CellDesc
    # the fp32 sources the packing kernels read, held with the buffer so that they outlive those
    # kernels without a host wait
    srcs: list = field(default_factory=list)


class NCA(nn.Module):
    """The cell update rule (reference model.py:304-355), computed by libnca_hip.so."""

    def __init__(self, cfg: NCAConfig):
        super().__init__()
        self.cfg = cfg
        C = cfg.channels
        self.register_buffer(
            "embed", make_embeddings(cfg.vocab_size, cfg.c_in, cfg.embedding, c_out=cfg.c_out)
        )
        if cfg.head in ("l2", "cosine"):
            lo = cfg.out_offset - cfg.in_offset
            self.register_buffer(
                "out_embed", self.embed[list(cfg.output_tokens)][:, lo: lo + cfg.c_out].clone()
            )
        pad_vec = torch.zeros(C)
        if cfg.padding == "wall":
            assert cfg.wall_token is not None, "wall padding needs wall_token"
            pad_vec[cfg.in_slice] = self.embed[cfg.wall_token]
        self.register_buffer("pad_vec", pad_vec)
        if cfg.perception != "kernels":
            raise ValueError(f"perception {cfg.perception!r} is not implemented (kernels only)")
        self.perceive = KernelPerception(C, cfg.heads, cfg.kernel_init)
        if cfg.update != "mlp":
            raise ValueError(f"update {cfg.update!r} is not implemented (mlp only)")
        self.update = MLPUpdate(self.perceive.out_dim, C, cfg.hidden, cfg.zero_init_update)
        if cfg.head == "mlp":
            self.head = nn.Conv2d(cfg.c_out, len(cfg.output_tokens), 1)
        self._packed: dict = {}

    # ------------------------------------------------------------------ checks
    def kernel_support(self) -> None:
        """Raise ValueError when the configuration is outside what the HIP kernels implement."""
        cfg = self.cfg
        bad = []
        if cfg.norm_groups:
            bad.append("norm_groups")
        if cfg.time_steps or cfg.n_tasks or cfg.c_task:
            bad.append("time / task embeddings")
        if cfg.project_update or cfg.noise_after_norm:
            bad.append("public-code update switches")
        if cfg.head not in ("mlp", "l2"):
            bad.append(f"head {cfg.head!r}")
        if cfg.heads != 4:
            bad.append(f"heads={cfg.heads}")
        if (cfg.channels, cfg.hidden) not in ((16, 128), (32, 256), (64, 256)):
            bad.append(f"C={cfg.channels} hidden={cfg.hidden}")
        if len(cfg.output_tokens) > 16:
            bad.append("more than 16 output tokens")
        if bad:
            raise ValueError("the HIP engine does not implement: " + ", ".join(bad))

    # ------------------------------------------------------------------ packed weights
    def cell_desc(self, precision: str) -> _lib.CellDesc:
        cfg = self.cfg
        return _lib.CellDesc(
            cfg.channels, cfg.heads, cfg.hidden, cfg.c_in, cfg.in_offset, cfg.c_out,
            cfg.out_offset, len(cfg.output_tokens), _lib.PADDING[cfg.padding], _lib.HEAD[cfg.head],
            _lib.PRECISION[precision],
        )

    def _head_tensors(self):
        if self.cfg.head == "mlp":
            return self.head.weight.reshape(len(self.cfg.output_tokens), -1), self.head.bias
        return self.out_embed, None

    def packed(self, precision: str = "fp32", device=None) -> _Packed:
        """The weights in the kernels' fragment layout, re-packed when a parameter changed."""
        if precision not in _lib.PRECISION:
            raise ValueError(f"precision {precision!r} (fp32 | bf16)")
        self.kernel_support()
        device = torch.device(device) if device is not None else self.pad_vec.device
        hw, hb = self._head_tensors()
        srcs = [self.perceive.weight, self.update.fc1.weight, self.update.fc1.bias,
                self.update.fc2.weight, self.update.fc2.bias, hw, hb, self.pad_vec]
        key = (precision, str(device)) + tuple(
            (None if t is None else (t.data_ptr(), t._version)) for t in srcs
        )
        cached = self._packed.get((precision, str(device)))
        if cached is not None and cached.key == key:
            return cached
        L = _lib.load()
        desc = self.cell_desc(precision)
        nbytes = L.nca_packed_weights_bytes(ctypes.byref(desc))
        if nbytes == 0:
            _lib.check(_lib.NCA_ERR_UNSUPPORTED, "nca_packed_weights_bytes")
        _lib.require_device(self.pad_vec.to(device))
        buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        flat = [None if t is None else t.detach().to(device, torch.float32).contiguous()
                for t in srcs]
        w = _lib.CellWeights(*[_lib.ptr(t) for t in flat])
        _lib.check(
            L.nca_pack_weights(ctypes.byref(desc), ctypes.byref(w), buf.data_ptr(),
                               _lib.stream_of(device)),
            "nca_pack_weights",
        )
        p = _Packed(key, buf, desc, flat)
        self._packed[(precision, str(device))] = p
        return p

    # ------------------------------------------------------------------ state construction
    @property
    def device(self) -> torch.device:
        return self.embed.device

    def clamp_values(self, inputs: torch.Tensor) -> torch.Tensor:
        """Token embeddings of the input grid (B, C_in, H, W) (reference model.py:378-382)."""
        return self.embed[inputs].permute(0, 3, 1, 2).contiguous()

    def apply_clamp(self, x, given4, clamp):
        """Reset the input channels of given cells (reference model.py:430-438)."""
        sl = self.cfg.in_slice
        x_in = torch.where(given4, clamp, x[:, sl])
        if sl.start == 0 and sl.stop == self.cfg.channels:
            return x_in
        return torch.cat([x[:, : sl.start], x_in, x[:, sl.stop:]], dim=1)

    def init_state(self, inputs, given, task_ids=None, generator=None):
        """(x, given4, clamp) for (B, H, W) token boards (reference model.py:384-412)."""
        cfg = self.cfg
        B, H, W = inputs.shape
        shape = (B, cfg.channels, H, W)
        dev = self.device
        draw = torch.rand if cfg.init_uniform else torch.randn
        noise = draw(shape, generator=generator, device=dev)
        given = given.to(dev)
        given4 = given[:, None]
        if dev.type == "cuda":
            # the scaling, the clamp values and their application in one launch (nca_init_state)
            sl = cfg.in_slice
            emb = self.embed.detach().to(torch.float32).contiguous()
            tok = inputs.to(dev, torch.int64).contiguous()
            g8 = (given.contiguous().view(torch.uint8) if given.dtype == torch.bool
                  else (given != 0).to(torch.uint8).contiguous())
            x = torch.empty(shape, dtype=torch.float32, device=dev)
            clamp = torch.empty((B, emb.shape[1], H, W), dtype=torch.float32, device=dev)
            if emb.shape[1] != sl.stop - sl.start:
                raise ValueError("the embedding width must equal the clamped input slice")
            _lib.check(_lib.load().nca_init_state(
                noise.data_ptr(), tok.data_ptr(), g8.data_ptr(), emb.data_ptr(), emb.shape[0], B,
                cfg.channels, emb.shape[1], sl.start, H * W, int(bool(cfg.init_uniform)),
                float(cfg.sigma_init), x.data_ptr(), clamp.data_ptr(), _lib.stream_of(dev)), "nca_init_state")
            return x, given4, clamp
        x = ((noise * 2 - 1) if cfg.init_uniform else noise) * cfg.sigma_init
        clamp = self.clamp_values(inputs.to(dev))
        return self.apply_clamp(x, given4, clamp), given4, clamp

    def target_embedding(self, targets):
        lo = self.cfg.out_offset - self.cfg.in_offset
        return self.embed[targets][..., lo: lo + self.cfg.c_out].permute(0, 3, 1, 2)

    def token_table(self, kind: str, device) -> torch.Tensor:
        """Small lookup tables on the device, uploaded once per device without a host wait:
        "tokens" (class index -> output token) and "index" (token -> class index, 0 for tokens
        that are no output; "index32" the same as int32)."""
        key = (kind, str(device))
        cache = self.__dict__.setdefault("_tables", {})
        t = cache.get(key)
        if t is None:
            if kind == "tokens":
                host = np.asarray(self.cfg.output_tokens, dtype=np.int64)
            else:
                host = np.zeros(self.cfg.vocab_size, dtype=np.int32 if kind == "index32" else np.int64)
                for i, tok in enumerate(self.cfg.output_tokens):
                    host[tok] = i
            t = cache[key] = _lib.upload(host, torch.device(device))
        return t

    def output_index(self, targets, dtype=torch.int64):
        """Class indices of target tokens (int64, or int32 with dtype=torch.int32)."""
        return self.token_table("index32" if dtype == torch.int32 else "index", targets.device)[targets]

    # ------------------------------------------------------------------ HIP operators
    def step(self, x, given4, clamp, fire_mask, noise=None, clock=None, precision="fp32"):
        """One step with an explicit fire mask (reference model.py:503-525)."""
        from .step import hip_step

        if clock is not None and self.cfg.time_steps:
            raise ValueError("time embeddings are not implemented")
        return hip_step(self, x, given4, clamp, fire_mask, noise, precision)

    def readout(self, x: torch.Tensor):
        """(conf_cell (B,H,W), conf_board (B,), argmax (B,H,W) int32) of fp32 states."""
        from .readout import readout

        return readout(self, x)

    def confidence(self, x):
        return self.readout(x)[0]

    def board_confidence(self, x):
        return self.readout(x)[1]

    def decode(self, x):
        idx = self.readout(x)[2].long()
        return self.token_table("tokens", x.device)[idx]

    def extra_repr(self) -> str:
        return ", ".join(f"{k}={v}" for k, v in self.cfg.to_dict().items())


# ---------------------------------------------------------------------- presets
# Maze vocabulary of the maze presets below: one-hot input channels wall / open / start / goal
# as tokens OPEN=0, WALL=1, START=2, GOAL=3; PATH=4 is an output-only token.
MAZE_OPEN, MAZE_WALL, MAZE_START, MAZE_GOAL, MAZE_PATH = 0, 1, 2, 3, 4

PRESETS: dict[str, dict] = {
    # the reference's maze presets (reference model.py:659-696), for their trained checkpoints
    "maze_ood": dict(vocab_size=4, channels=16, c_in=16, c_out=2, output_tokens=(0, 1),
                     perception="kernels", hidden_from_perception=True, heads=4, padding="wall",
                     wall_token=2, update="mlp", expansion=2, norm_groups=0, sigma_init=0.15,
                     fire_rate=0.8, head="l2", embedding="onehot"),
    "maze_hard": dict(vocab_size=5, channels=32, c_in=32, c_out=3, output_tokens=(0, 1),
                      perception="kernels", hidden_from_perception=True, heads=4, padding="wall",
                      wall_token=2, update="mlp", expansion=2, norm_groups=0, sigma_init=0.25,
                      fire_rate=0.8, head="l2", embedding="onehot"),
    # C=16 maze cell: 4 one-hot input channels (open / wall / start / goal), 64 features,
    # MLP 64 -> 128 -> 16, 2-class (open / path) mlp readout on channels 4..7
    "maze_c16": dict(vocab_size=5, channels=16, c_in=4, c_out=4, out_offset=4,
                     output_tokens=(MAZE_OPEN, MAZE_PATH), hidden_from_perception=True, heads=4,
                     padding="wall", wall_token=MAZE_WALL, expansion=2, sigma_init=0.0,
                     fire_rate=0.5, head="mlp", embedding="onehot_inputs", kernel_init="fixed"),
    # C=32 hard-maze cell: MLP 128 -> 256 -> 32
    "maze_hard_c32": dict(vocab_size=5, channels=32, c_in=4, c_out=4, out_offset=4,
                          output_tokens=(MAZE_OPEN, MAZE_PATH), hidden_from_perception=True,
                          heads=4, padding="wall", wall_token=MAZE_WALL, expansion=2,
                          sigma_init=0.0, fire_rate=0.8, head="mlp", embedding="onehot_inputs",
                          kernel_init="fixed"),
    # C=64 Sudoku cell: 10 one-hot input channels (0 = empty, 1..9), 256 features,
    # MLP 256 -> 256 -> 64, 9-digit mlp readout on channels 10..25, wrap padding
    # (the reference's Sudoku presets pad with wrap, model.py:706)
    "sudoku_c64": dict(vocab_size=10, channels=64, c_in=10, c_out=16, out_offset=10,
                       output_tokens=tuple(range(1, 10)), hidden_from_perception=False, heads=4,
                       padding="wrap", wall_token=None, expansion=4, sigma_init=0.0,
                       fire_rate=0.5, head="mlp", embedding="onehot", kernel_init="fixed"),
}


def build_model(preset: str | None = None, **overrides) -> NCA:
    d = dict(PRESETS[preset]) if preset else {}
    d.update(overrides)
    d["output_tokens"] = tuple(d["output_tokens"])
    return NCA(NCAConfig(**d))


def init_weights(model: NCA, seed: int = 0, std: float = 0.02, zero_last: bool = True) -> NCA:
    """Synthetic weights: N(0, std) for every fc and head weight, zero biases, in the fixed
    order fc1.weight, fc2.weight, head.weight from `torch.Generator(seed)`; fc2 zero when
    `zero_last` (the do-nothing rule; parity runs perturb it)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in (("fc1", model.update.fc1), ("fc2", model.update.fc2)):
            w = torch.randn(p.weight.shape, generator=g) * std
            p.weight.copy_(w if not (name == "fc2" and zero_last) else torch.zeros_like(w))
            p.bias.zero_()
        if model.cfg.head == "mlp":
            model.head.weight.copy_(torch.randn(model.head.weight.shape, generator=g) * std)
            model.head.bias.zero_()
    return model


@dataclass
class ModelSpec:
    preset: str | None = None
    overrides: dict = field(default_factory=dict)

    def build(self) -> NCA:
        return build_model(self.preset, **self.overrides)

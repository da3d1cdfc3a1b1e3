"""Seeded synthetic workloads for the verify + commit path.

Five named workloads (sizes in the table below) generate the inputs a GDN layer
sees under speculative decoding:

* q, k: bf16 N(0, 1), then L2-normalised per head (eps 1e-6);
* v: bf16 N(0, 1); beta = sigmoid(N(0, 1)) fp32; g = -softplus(N(0, 1)) fp32;
* FP32 checkpoint pages N(0, 0.1); page 0 is the null page;
* accepted lengths uniform in {0..Q}, geometric(p=0.3) capped at Q, or all Q;
* align mode: block size 64, positions C ~ U[0, 8192); a seeded quarter of the
  rows with n >= 1 is moved so that the next block boundary lies 1..n tokens
  ahead (so about 25% of the rows cross a boundary); each row owns distinct
  pages for its source column and the next one; a few rows are padded with -1.

| name              | layers | rows | H  | HV | K=V | Q | mode  | accept    |
|-------------------|--------|------|----|----|-----|---|-------|-----------|
| plumbing_b4       | 1      | 4    | 2  | 4  | 64  | 4 | none  | uniform   |
| pool512_b64       | 1      | 64   | 16 | 32 | 128 | 4 | none  | uniform   |
| align_b256        | 1      | 256  | 16 | 32 | 128 | 4 | align | uniform   |
| decode_q1_b256    | 1      | 256  | 16 | 32 | 128 | 1 | none  | all       |
| skewed_q8_b256    | 1      | 256  | 16 | 32 | 128 | 8 | none  | geometric |
| decode_loop_l48   | 48     | 128  | 16 | 32 | 128 | 4 | align | uniform   |
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

import torch

NULL_PAGE = 0


@dataclass(frozen=True)
class WorkloadSpec:
    name: str
    layers: int
    rows: int
    key_heads: int
    value_heads: int
    key_dim: int
    value_dim: int
    window: int
    align: bool = False
    block_size: int = 64
    max_position: int = 8192
    crossing_fraction: float = 0.25
    padded_rows: int = 0
    accept: str = "uniform"  # uniform | geometric | all
    steps: int = 1
    pool_pages: int | None = None  # none mode: pool size (page 0 is null)
    conv_kernel: int = 4
    state_dtype: torch.dtype = torch.float32
    act_dtype: torch.dtype = torch.bfloat16


SPECS = {
    "plumbing_b4": WorkloadSpec("plumbing_b4", 1, 4, 2, 4, 64, 64, 4),
    "pool512_b64": WorkloadSpec("pool512_b64", 1, 64, 16, 32, 128, 128, 4, pool_pages=512),
    "align_b256": WorkloadSpec("align_b256", 1, 256, 16, 32, 128, 128, 4, align=True, padded_rows=6),
    "decode_q1_b256": WorkloadSpec("decode_q1_b256", 1, 256, 16, 32, 128, 128, 1, accept="all", pool_pages=512),
    "skewed_q8_b256": WorkloadSpec("skewed_q8_b256", 1, 256, 16, 32, 128, 128, 8, accept="geometric", pool_pages=512),
    "decode_loop_l48": WorkloadSpec("decode_loop_l48", 48, 128, 16, 32, 128, 128, 4, align=True, steps=64, padded_rows=2),
}


def get_spec(name: str, **overrides) -> WorkloadSpec:
    return replace(SPECS[name], **overrides) if overrides else SPECS[name]


@dataclass
class LayerInputs:
    q: torch.Tensor  # [1, T, H, K]
    k: torch.Tensor  # [1, T, H, K]
    v: torch.Tensor  # [1, T, HV, V]
    g: torch.Tensor  # [T, HV] fp32 log-decay
    beta: torch.Tensor  # [T, HV] fp32


@dataclass
class StepMeta:
    query_start_loc: torch.Tensor  # [B + 1] int32
    state_indices: torch.Tensor  # [B] int32 (column view of a [B, Q] table)
    request_indices: torch.Tensor  # [B] int64
    accepted: torch.Tensor  # [B] int32, indexed by request
    idx_mapping: torch.Tensor  # [B] int32, request -> persistent slot
    block_table: torch.Tensor | None = None  # [B, W] int32
    num_computed: torch.Tensor | None = None  # [B] int32
    block_size: int | None = None


@dataclass
class Workload:
    spec: WorkloadSpec
    num_pages: int
    checkpoints: list  # per layer [NB, HV, V, K]
    conv_states: list  # per layer [NB, conv_dim, hist + Q - 1]
    inputs: list  # per layer LayerInputs
    meta: StepMeta
    extras: dict = field(default_factory=dict)

    @property
    def tokens(self) -> int:
        return int(self.meta.query_start_loc[-1])

    def to(self, device) -> "Workload":
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        m = self.meta
        meta = StepMeta(
            mv(m.query_start_loc), None, mv(m.request_indices), mv(m.accepted), mv(m.idx_mapping),
            mv(m.block_table), mv(m.num_computed), m.block_size,
        )
        table = self.extras["state_table"].to(device)
        meta.state_indices = table[:, 0]
        return Workload(
            self.spec,
            self.num_pages,
            [c.to(device) for c in self.checkpoints],
            [c.to(device) for c in self.conv_states],
            [LayerInputs(mv(i.q), mv(i.k), mv(i.v), mv(i.g), mv(i.beta)) for i in self.inputs],
            meta,
            {**self.extras, "state_table": table},
        )


def _l2(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) + 1e-6)


def sample_accepted(spec: WorkloadSpec, rows: int, gen: torch.Generator) -> torch.Tensor:
    Q = spec.window
    if spec.accept == "all":
        return torch.full((rows,), Q, dtype=torch.int32)
    if spec.accept == "geometric":
        # failures before the first success, p = 0.3, capped at Q
        u = torch.rand(rows, generator=gen, dtype=torch.float64).clamp_min(1e-300)
        n = torch.floor(torch.log(u) / torch.log(torch.tensor(0.7, dtype=torch.float64)))
        return n.clamp(max=Q).to(torch.int32)
    return torch.randint(0, Q + 1, (rows,), generator=gen, dtype=torch.int32)


def make_layer_inputs(spec: WorkloadSpec, tokens: int, gen: torch.Generator, device="cpu") -> LayerInputs:
    H, HV, K, V = spec.key_heads, spec.value_heads, spec.key_dim, spec.value_dim
    q = _l2(torch.randn(1, tokens, H, K, generator=gen, device=device).to(spec.act_dtype)).to(spec.act_dtype)
    k = _l2(torch.randn(1, tokens, H, K, generator=gen, device=device).to(spec.act_dtype)).to(spec.act_dtype)
    v = torch.randn(1, tokens, HV, V, generator=gen, device=device).to(spec.act_dtype)
    beta = torch.sigmoid(torch.randn(tokens, HV, generator=gen, device=device))
    g = -torch.nn.functional.softplus(torch.randn(tokens, HV, generator=gen, device=device))
    return LayerInputs(q, k, v, g, beta)


def make_align_meta(spec: WorkloadSpec, gen: torch.Generator, accepted: torch.Tensor):
    """Positions, block table and source pages for align mode.

    Row r owns distinct pages for the column holding its state ((C - 1) // Bk)
    and the columns its positions can reach over ``spec.steps`` windows; every
    other column is the null page.
    """
    B, Bk, Q = spec.rows, spec.block_size, spec.window
    C = torch.randint(0, spec.max_position, (B,), generator=gen, dtype=torch.int64)
    # Only rows with n >= 1 can cross; pick among them so that about
    # `crossing_fraction` of all rows do.
    movable = max(float((accepted >= 1).float().mean()), 1e-6)
    pick = torch.rand(B, generator=gen) < min(1.0, spec.crossing_fraction / movable)
    for r in range(B):
        n = int(accepted[r])
        if pick[r] and n >= 1:
            ahead = int(torch.randint(1, n + 1, (1,), generator=gen))
            base = max(int(C[r]) // Bk, 1) * Bk
            C[r] = base - ahead  # next boundary is `ahead` tokens away
    width = spec.max_position // Bk + 2 + (Q * spec.steps) // Bk + 1
    table = torch.zeros(B, width, dtype=torch.int32)
    src_col = torch.clamp(C - 1, min=0) // Bk
    pages_per_row = 2 + -(-Q * spec.steps // Bk)
    for r in range(B):
        a = int(src_col[r])
        for j in range(pages_per_row):
            if a + j < width:
                table[r, a + j] = 1 + pages_per_row * r + j
    num_pages = 1 + pages_per_row * B
    return C.to(torch.int32), table, src_col, num_pages


def make_workload(name: str, *, seed: int = 0, gen_device="cpu", **overrides) -> Workload:
    spec = get_spec(name, **overrides)
    gen = torch.Generator(device="cpu").manual_seed(seed)
    B, Q, HV, K, V, H = spec.rows, spec.window, spec.value_heads, spec.key_dim, spec.value_dim, spec.key_heads
    accepted = sample_accepted(spec, B, gen)
    tokens = B * Q
    qsl = torch.arange(B + 1, dtype=torch.int32) * Q
    state_table = torch.zeros(B, Q, dtype=torch.int32)
    extras = {}
    if spec.align:
        C, table, src_col, num_pages = make_align_meta(spec, gen, accepted)
        src = table[torch.arange(B), src_col]
        block_table, num_computed = table, C
        extras["source_col"] = src_col
    else:
        num_pages = spec.pool_pages or (2 * B + 1)
        perm = torch.randperm(num_pages - 1, generator=gen)[:B] + 1
        src = perm.to(torch.int32)
        block_table = num_computed = None
    if spec.padded_rows:
        pad = torch.randperm(B, generator=gen)[: spec.padded_rows]
        src = src.clone()
        src[pad] = -1
        extras["padded_rows"] = pad
    state_table[:, 0] = src
    request_indices = torch.arange(B, dtype=torch.int64)
    idx_mapping = torch.arange(B, dtype=torch.int32)
    meta = StepMeta(
        qsl, state_table[:, 0], request_indices, accepted, idx_mapping, block_table, num_computed,
        spec.block_size if spec.align else None,
    )
    extras["state_table"] = state_table
    dgen = gen if gen_device == "cpu" else torch.Generator(device=gen_device).manual_seed(seed + 1)
    checkpoints, convs, inputs = [], [], []
    conv_dim = 2 * H * K + HV * V
    conv_len = spec.conv_kernel - 1 + Q - 1
    for _ in range(spec.layers):
        ck = torch.randn(num_pages, HV, V, K, generator=dgen, device=gen_device, dtype=torch.float32) * 0.1
        checkpoints.append(ck.to(spec.state_dtype))
        convs.append(torch.randn(num_pages, conv_dim, conv_len, generator=dgen, device=gen_device).to(spec.act_dtype))
        inputs.append(make_layer_inputs(spec, tokens, dgen, device=gen_device))
    return Workload(spec, num_pages, checkpoints, convs, inputs, meta, extras)


def advance_align(meta: StepMeta, plan_lengths: torch.Tensor, plan_final: torch.Tensor) -> StepMeta:
    """Carry align-mode state to the next speculative step.

    Rows whose commit was valid advance C by the committed length and continue
    from the final page; other rows keep their position and source page.
    """
    n = plan_lengths.to(meta.num_computed.dtype)
    committed = n > 0
    new_c = meta.num_computed + n
    src = torch.where(committed, plan_final.to(meta.state_indices.dtype), meta.state_indices)
    table = torch.zeros(meta.state_indices.shape[0], 1, dtype=meta.state_indices.dtype, device=meta.state_indices.device)
    table[:, 0] = src
    return replace(meta, num_computed=new_c, state_indices=table[:, 0])


__all__ = [
    "SPECS",
    "WorkloadSpec",
    "LayerInputs",
    "StepMeta",
    "Workload",
    "get_spec",
    "make_workload",
    "make_layer_inputs",
    "sample_accepted",
    "advance_align",
]

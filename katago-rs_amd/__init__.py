"""Python binding of libkgx (include/kgx.h), the KataGo forward pass on MI355X.

This mirrors the reference backend's interface (crates/katago-nn-burn/src/backend.rs): a loaded model
(`Net`, NeuralNet::load_model_file), a device handle (`Handle`, create_compute_context +
create_compute_handle), the raw forward pass (`Handle.forward`, run_network) and `Handle.get_output`
(copy_inputs / run_network / copy_outputs). It calls the C ABI through ctypes; there is no other compute path,
and a missing or unbuilt library is an error.

The package directory name is not a Python identifier; import it with
``importlib.import_module("katago-rs_amd")`` after putting the repository root on ``sys.path``.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkgx.so")
CSRC = os.path.join(HERE, "csrc")

PRECISION_F32 = 0
PRECISION_F16 = 1
PRECISION_BF16 = 2
PRECISIONS = {"f32": PRECISION_F32, "f16": PRECISION_F16, "bf16": PRECISION_BF16}

HW = 361
MAX_POLICY = 362

# Every symbol the C header declares (include/kgx.h).
EXPORTS = [
    "kg_version", "kg_last_error", "kg_device_count", "kg_device_open", "kg_net_load", "kg_net_free", "kg_net_desc",
    "kg_handle_create", "kg_handle_free", "kg_handle_set_batch_buckets", "kg_padded_batch_size",
    "kg_copy_with_symmetry",
    "kg_handle_is_using_fp16", "kg_forward", "kg_handle_device_buffers", "kg_run", "kg_sync", "kg_handle_stream",
    "kg_get_output", "kg_profile_enable", "kg_profile_reset", "kg_profile_read",
    "kg_model_version_features", "kg_meta_encoder_channels", "kg_copy_outputs", "kg_run_static",
    "kg_get_output_async", "kg_wait", "kg_get_output_eval", "kg_post_outputs",
    "kg_conv_geometry", "kg_conv_tile_of", "kg_conv_weight_load", "kg_conv_weight_chunk", "kg_junction_tile_of", "kg_gpool_tile_of", "kg_l2_touch_line", "kg_rmsnorm_rows_of",
    "kg_featurize", "kg_featurize_rows", "kg_evaluate_positions",
]
# Completion callback of kg_get_output_async: (user, status).
DONE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int)

_lib = None


def build(jobs: int = 4):
    """Compiles libkgx.so for gfx950 with hipcc (katago-rs_amd/csrc/Makefile)."""
    subprocess.run(["make", "-C", CSRC, f"-j{jobs}", "-s"], check=True)


class KgError(RuntimeError):
    pass


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 128),
        ("model_version", ctypes.c_int),
        ("num_input_channels", ctypes.c_int),
        ("num_input_global_channels", ctypes.c_int),
        ("num_input_meta_channels", ctypes.c_int),
        ("num_policy_channels", ctypes.c_int),
        ("num_value_channels", ctypes.c_int),
        ("num_score_value_channels", ctypes.c_int),
        ("num_ownership_channels", ctypes.c_int),
        ("trunk_num_channels", ctypes.c_int),
        ("trunk_num_blocks", ctypes.c_int),
        ("num_parameters", ctypes.c_long),
        ("post_process_params", ctypes.c_float * 7),
        ("output_row_len", ctypes.c_int),
    ]


class RowInput(ctypes.Structure):
    _fields_ = [
        ("row_spatial", ctypes.c_void_p),
        ("row_global", ctypes.c_void_p),
        ("row_meta", ctypes.c_void_p),
        ("symmetry", ctypes.c_int),
        ("policy_optimism", ctypes.c_float),
    ]


class PostInput(ctypes.Structure):
    """kg_post_input: NNEvaluator's per-row inputs of the output post-processing (nneval.rs:1197-1500)."""
    _fields_ = [
        ("legal", ctypes.c_void_p),
        ("white_to_move", ctypes.c_int),
        ("board_x_size", ctypes.c_int),
        ("board_y_size", ctypes.c_int),
        ("nn_policy_temperature", ctypes.c_float),
        ("enable_passing_hacks", ctypes.c_int),
        ("no_result_allowed", ctypes.c_int),
    ]


class Position(ctypes.Structure):
    """kg_position: a position for the device featurizer (fill_row_v7's inputs, nninputs.rs:1336-1800)."""
    _fields_ = [(f, ctypes.c_int) for f in (
        "x_size", "y_size", "next_player", "ko_loc", "encore_phase", "ko_rule", "scoring_rule", "tax_rule",
        "multi_stone_suicide_legal", "has_button", "pass_would_end_phase", "history_turns", "num_moves")] + [
        ("move_loc", ctypes.c_int * 5), ("move_player", ctypes.c_int * 5), ("self_komi", ctypes.c_float),
        ("playout_doubling_advantage", ctypes.c_double), ("color", ctypes.c_ubyte * 361),
        ("area", ctypes.c_ubyte * 361), ("encore_start", ctypes.c_ubyte * 361), ("marks", ctypes.c_ubyte * 361)]


def make_positions(items):
    """A ctypes array of Position from dicts with keys meta (x_size, y_size, next_player, ko_loc, encore_phase,
    ko_rule, scoring_rule, tax_rule, multi_stone_suicide_legal, has_button, pass_would_end_phase, history_turns,
    num_moves), color, marks, area, enc ([361] uint8, index x + y * x_size), moves ([10]: loc, player per move),
    self_komi and pda."""
    arr = (Position * len(items))()
    names = [f for f, _ in Position._fields_[:13]]
    for i, it in enumerate(items):
        p = arr[i]
        for f, v in zip(names, it["meta"]):
            setattr(p, f, int(v))
        mv = np.asarray(it["moves"], np.int32)
        for k in range(5):
            p.move_loc[k] = int(mv[2 * k])
            p.move_player[k] = int(mv[2 * k + 1])
        p.self_komi = float(it["self_komi"])
        p.playout_doubling_advantage = float(it["pda"])
        for f, key in (("color", "color"), ("area", "area"), ("encore_start", "enc"), ("marks", "marks")):
            ctypes.memmove(getattr(p, f), np.ascontiguousarray(it[key], np.uint8).ctypes.data, 361)
    return arr


def featurize_rows(positions, nn_x: int = 19, nn_y: int = 19, nhwc: bool = False, symmetry=None, device: int = 0):
    """The device featurizer between host buffers (kg_featurize_rows): ([n, 22 * nn_x * nn_y], [n, 19]) float32."""
    n = len(positions)
    bin_ = np.empty((n, 22 * nn_x * nn_y), np.float32)
    glob = np.empty((n, 19), np.float32)
    sym = None if symmetry is None else np.ascontiguousarray(symmetry, np.int32)
    _check(lib().kg_featurize_rows(device, n, positions, nn_x, nn_y, int(bool(nhwc)), _ptr(sym), _ptr(bin_),
                                   _ptr(glob)))
    return bin_, glob


class ConvGeometry(ctypes.Structure):
    """kg_conv_geometry_t: the launch geometry of the 16-bit implicit-GEMM convolution of given shapes."""
    _fields_ = [(f, ctypes.c_int) for f in (
        "grid", "threads", "tile_rows", "tile_cols", "stage_channels", "pixel_tiles", "col_tiles", "pairs",
        "weights_direct", "weight_rows", "waves", "direct_instructions", "direct_per_wave")]


class NNOutput(ctypes.Structure):
    _fields_ = [
        ("policy_probs", ctypes.c_float * MAX_POLICY),
        ("white_win_prob", ctypes.c_float),
        ("white_loss_prob", ctypes.c_float),
        ("white_no_result_prob", ctypes.c_float),
        ("white_score_mean", ctypes.c_float),
        ("white_score_mean_sq", ctypes.c_float),
        ("white_lead", ctypes.c_float),
        ("var_time_left", ctypes.c_float),
        ("shortterm_winloss_error", ctypes.c_float),
        ("shortterm_score_error", ctypes.c_float),
        ("white_owner_map", ctypes.c_void_p),
    ]


def lib():
    """The loaded libkgx.so. Raises if it has not been built: there is no fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise KgError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (make -C {CSRC})")
        L = ctypes.CDLL(LIB_PATH)
        vp, ci, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.kg_version.restype = ctypes.c_char_p
        L.kg_last_error.restype = ctypes.c_char_p
        L.kg_device_count.argtypes = [ctypes.POINTER(ci)]
        L.kg_device_open.argtypes = [ci]
        L.kg_net_load.argtypes = [vp, ctypes.c_size_t, ctypes.c_char_p, ctypes.POINTER(vp)]
        L.kg_net_free.argtypes = [vp]
        L.kg_net_desc.argtypes = [vp, ctypes.POINTER(ModelDesc)]
        L.kg_handle_create.argtypes = [vp, ci, ci, ci, ci, ci, ci, ctypes.POINTER(vp)]
        L.kg_handle_free.argtypes = [vp]
        L.kg_handle_set_batch_buckets.argtypes = [vp, vp, ci]
        L.kg_padded_batch_size.argtypes = [vp, ci, ci, ci]
        L.kg_copy_with_symmetry.argtypes = [vp, vp, ci, ci, ci, ci, ci]
        L.kg_handle_is_using_fp16.argtypes = [vp]
        L.kg_forward.argtypes = [vp, ci, vp, vp, vp, vp]
        L.kg_handle_device_buffers.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.POINTER(vp),
                                               ctypes.POINTER(vp)]
        L.kg_run.argtypes = [vp, ci, vp]
        L.kg_sync.argtypes = [vp]
        L.kg_run_static.argtypes = [vp, ci]
        L.kg_get_output_async.argtypes = [vp, ci, ctypes.POINTER(RowInput), ctypes.POINTER(NNOutput), DONE_FN, vp]
        L.kg_wait.argtypes = [vp]
        L.kg_handle_stream.argtypes = [vp]
        L.kg_handle_stream.restype = vp
        L.kg_get_output.argtypes = [vp, ci, ctypes.POINTER(RowInput), ctypes.POINTER(NNOutput)]
        L.kg_profile_enable.argtypes = [vp, ci]
        L.kg_profile_reset.argtypes = [vp]
        L.kg_profile_read.argtypes = [vp, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_long),
                                      ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_double), ci]
        L.kg_model_version_features.argtypes = [ci, ctypes.POINTER(ci), ctypes.POINTER(ci), ctypes.POINTER(ci)]
        L.kg_meta_encoder_channels.argtypes = [ci, ctypes.POINTER(ci)]
        L.kg_copy_outputs.argtypes = [vp, ci, ci, ci, ci, vp, vp, ctypes.POINTER(NNOutput)]
        L.kg_get_output_eval.argtypes = [vp, ci, ctypes.POINTER(RowInput), ctypes.POINTER(PostInput),
                                         ctypes.POINTER(NNOutput)]
        L.kg_post_outputs.argtypes = [vp, ci, vp, vp, vp, ctypes.POINTER(PostInput), ctypes.POINTER(NNOutput)]
        L.kg_featurize.argtypes = [vp, ci, ctypes.POINTER(Position), vp]
        L.kg_featurize_rows.argtypes = [ci, ci, ctypes.POINTER(Position), ci, ci, ci, vp, vp, vp]
        L.kg_evaluate_positions.argtypes = [vp, ci, ctypes.POINTER(Position), vp, vp, ctypes.POINTER(PostInput),
                                            ctypes.POINTER(NNOutput)]
        L.kg_conv_geometry.argtypes = [ci, ci, ci, ci, ci, ctypes.POINTER(ConvGeometry)]
        L.kg_conv_tile_of.argtypes = [ci, ci, ci, ci, ci, ci, ctypes.POINTER(ci), ctypes.POINTER(ci)]
        L.kg_conv_weight_load.argtypes = [ci, ci, ci, ci, ci, ci, ci] + [ctypes.POINTER(ci)] * 4
        L.kg_conv_weight_chunk.argtypes = [ci, ci]
        L.kg_junction_tile_of.argtypes = [ci, ci, ctypes.POINTER(ci), ctypes.POINTER(ci)]
        L.kg_gpool_tile_of.argtypes = [ci, ci, ci, ci] + [ctypes.POINTER(ci)] * 4
        L.kg_l2_touch_line.argtypes = [ci, ci, ci, ctypes.POINTER(ci)]
        L.kg_rmsnorm_rows_of.argtypes = [ci, ci, ci, ci] + [ctypes.POINTER(ci)] * 3
        _ = cf
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise KgError(lib().kg_last_error().decode())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def version() -> str:
    return lib().kg_version().decode()


def device_count() -> int:
    c = ctypes.c_int()
    _check(lib().kg_device_count(ctypes.byref(c)))
    return c.value


def padded_batch_size(buckets, n, max_batch) -> int:
    b = np.ascontiguousarray(buckets, np.int32)
    return lib().kg_padded_batch_size(_ptr(b), len(b), n, max_batch)


def copy_with_symmetry(src, symmetry: int, reverse: bool = False) -> np.ndarray:
    """copy_inputs_with_symmetry (reverse False) / copy_outputs_with_symmetry (reverse True) of one row of
    [C, H, W] float planes (crates/katago-core/src/neuralnet/nninputs.rs:756-879), through the library."""
    a = np.ascontiguousarray(src, np.float32)
    if a.ndim != 3:
        raise ValueError("copy_with_symmetry: src must be [C, H, W]")
    out = np.empty_like(a)
    _check(lib().kg_copy_with_symmetry(_ptr(a), _ptr(out), a.shape[0], a.shape[1], a.shape[2], int(symmetry),
                                       int(bool(reverse))))
    return out


def conv_geometry(ks: int, ic: int, oc: int, split: bool, pixels: int) -> dict:
    """The launch geometry of the 16-bit implicit-GEMM convolution ks x ks, ic -> oc, over `pixels` pixels."""
    g = ConvGeometry()
    _check(lib().kg_conv_geometry(ks, ic, oc, int(split), pixels, ctypes.byref(g)))
    return {f: getattr(g, f) for f, _ in ConvGeometry._fields_}


def junction_tile_of(pixels: int, workgroup: int):
    """(workgroups of the junction launch over `pixels` pixels, the 48-pixel tile of `workgroup` or -1)."""
    grid, tile = ctypes.c_int(), ctypes.c_int()
    _check(lib().kg_junction_tile_of(pixels, workgroup, ctypes.byref(grid), ctypes.byref(tile)))
    return grid.value, tile.value


def gpool_tile_of(pixels: int, gpool_channels: int, regular_channels: int, workgroup: int):
    """(workgroups of the gpool tile launch, the 192-pixel tile of `workgroup` or -1, its first regular channel,
    its channel count)."""
    out = [ctypes.c_int() for _ in range(4)]
    _check(lib().kg_gpool_tile_of(pixels, gpool_channels, regular_channels, workgroup, *[ctypes.byref(o) for o in out]))
    return tuple(o.value for o in out)


def l2_touch_line(grid: int, workgroup: int, thread: int) -> int:
    """The 128-byte line of the next op's weights that a thread of a `grid`-workgroup launch touches into L2."""
    line = ctypes.c_int()
    _check(lib().kg_l2_touch_line(grid, workgroup, thread, ctypes.byref(line)))
    return line.value


def rmsnorm_rows_of(rows: int, channels: int, region: int, workgroup: int):
    """(workgroups of the RMSNorm launch, the first row of `workgroup`, its row count) when the rows were written in
    row tiles of `region` rows on XCD (tile mod 8)."""
    out = [ctypes.c_int() for _ in range(3)]
    _check(lib().kg_rmsnorm_rows_of(rows, channels, region, workgroup, *[ctypes.byref(o) for o in out]))
    return tuple(o.value for o in out)


def conv_tile_of(ks: int, ic: int, oc: int, split: bool, pixels: int, workgroup: int):
    """(pixel tile, column tile) of a workgroup of that convolution's launch; (-1, -1) if it exits at once."""
    mt, nt = ctypes.c_int(), ctypes.c_int()
    _check(lib().kg_conv_tile_of(ks, ic, oc, int(split), pixels, workgroup, ctypes.byref(mt), ctypes.byref(nt)))
    return mt.value, nt.value


def conv_weight_load(ks: int, ic: int, oc: int, split: bool, q: int, wave: int, lane: int):
    """(src row, src chunk, dst row, dst chunk) of direct weight load q of (wave, lane); dst row -1: spare."""
    r = [ctypes.c_int() for _ in range(4)]
    _check(lib().kg_conv_weight_load(ks, ic, oc, int(split), q, wave, lane, *[ctypes.byref(x) for x in r]))
    return tuple(x.value for x in r)


def conv_weight_chunk(row: int, chunk: int) -> int:
    return lib().kg_conv_weight_chunk(row, chunk)


def model_version_features(model_version: int):
    """(inputs version, spatial features, global features) of a model version (NNModelVersion)."""
    iv, sp, gl = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(lib().kg_model_version_features(int(model_version), ctypes.byref(iv), ctypes.byref(sp), ctypes.byref(gl)))
    return iv.value, sp.value, gl.value


def meta_encoder_channels(meta_encoder_version: int) -> int:
    c = ctypes.c_int()
    _check(lib().kg_meta_encoder_channels(int(meta_encoder_version), ctypes.byref(c)))
    return c.value


def _output_dict(o, own):
    return {
        "policy": np.ctypeslib.as_array(o.policy_probs).copy(),
        "white_win_prob": o.white_win_prob, "white_loss_prob": o.white_loss_prob,
        "white_no_result_prob": o.white_no_result_prob, "white_score_mean": o.white_score_mean,
        "white_score_mean_sq": o.white_score_mean_sq, "white_lead": o.white_lead,
        "var_time_left": o.var_time_left, "shortterm_winloss_error": o.shortterm_winloss_error,
        "shortterm_score_error": o.shortterm_score_error, "ownership": own,
    }


def copy_outputs(raw, P: int, S: int, model_version: int, symmetry, policy_optimism, want_ownership=True):
    """copy_outputs (crates/katago-nn-burn/src/backend.rs:622-731) on the host: raw rows [n, P*362 + 3 + S + 361]
    to a list of dicts of NNOutput fields."""
    raw = np.ascontiguousarray(raw, np.float32)
    n = raw.shape[0]
    if raw.shape != (n, P * 362 + 3 + S + HW):
        raise ValueError(f"raw rows must be [n, {P * 362 + 3 + S + HW}], got {raw.shape}")
    sym = np.ascontiguousarray(np.broadcast_to(symmetry, (n,)), np.int32)
    opt = np.ascontiguousarray(np.broadcast_to(policy_optimism, (n,)), np.float32)
    outs = (NNOutput * n)()
    owners = [np.zeros(HW, np.float32) if want_ownership else None for _ in range(n)]
    for i in range(n):
        outs[i].white_owner_map = None if owners[i] is None else _ptr(owners[i]).value
    _check(lib().kg_copy_outputs(_ptr(raw), n, P, S, model_version, _ptr(sym), _ptr(opt), outs))
    return [_output_dict(outs[i], owners[i]) for i in range(n)]


class Net:
    """A parsed KataGo model (NeuralNet::load_model_file)."""

    def __init__(self, model_bytes: bytes, expected_sha256: str = ""):
        self._h = None
        h = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(model_bytes, len(model_bytes))
        _check(lib().kg_net_load(buf, len(model_bytes), expected_sha256.encode(), ctypes.byref(h)))
        self._h = h
        d = ModelDesc()
        _check(lib().kg_net_desc(self._h, ctypes.byref(d)))
        self.desc = d
        self.name = d.name.decode()
        self.version = d.model_version
        self.P = d.num_policy_channels
        self.S = d.num_score_value_channels
        self.row_len = d.output_row_len
        self.num_input_channels = d.num_input_channels
        self.num_global = d.num_input_global_channels
        self.num_meta = d.num_input_meta_channels

    def __del__(self):
        if self._h:
            lib().kg_net_free(self._h)
            self._h = None


class Handle:
    """A device replica of a net (create_compute_context + create_compute_handle) for up to max_batch rows."""

    def __init__(self, net: Net, max_batch: int, precision="f16", device: int = 0, nn_x_len: int = 19,
                 nn_y_len: int = 19, inputs_use_nhwc: bool = False):
        self._h = None
        self.net = net
        self.max_batch = max_batch
        p = PRECISIONS[precision] if isinstance(precision, str) else int(precision)
        h = ctypes.c_void_p()
        _check(lib().kg_handle_create(net._h, device, max_batch, p, nn_x_len, nn_y_len, int(inputs_use_nhwc),
                                      ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().kg_handle_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def is_using_fp16(self) -> bool:
        return bool(lib().kg_handle_is_using_fp16(self._h))

    def set_batch_buckets(self, buckets):
        b = np.ascontiguousarray(buckets, np.int32)
        _check(lib().kg_handle_set_batch_buckets(self._h, _ptr(b), len(b)))

    def forward(self, spatial, glob, meta=None) -> np.ndarray:
        """Raw output rows [n, row_len] for inputs spatial [n, C, 19, 19], glob [n, G] (meta [n, 192])."""
        n = spatial.shape[0]
        spatial = np.ascontiguousarray(spatial, np.float32)
        glob = np.ascontiguousarray(glob, np.float32)
        meta = None if meta is None else np.ascontiguousarray(meta, np.float32)
        # kg_forward reads n rows of each input: shapes are checked here, where the arrays' sizes are known.
        net = self.net
        if spatial.shape != (n, net.num_input_channels, 19, 19):
            raise ValueError(f"spatial must be [n, {net.num_input_channels}, 19, 19], got {spatial.shape}")
        if glob.shape != (n, net.num_global):
            raise ValueError(f"glob must be [n, {net.num_global}], got {glob.shape}")
        if meta is not None and meta.shape != (n, net.num_meta):
            raise ValueError(f"meta must be [n, {net.num_meta}], got {meta.shape}")
        out = np.empty((n, self.net.row_len), np.float32)
        _check(lib().kg_forward(self._h, n, _ptr(spatial), _ptr(glob), _ptr(meta), _ptr(out)))
        return out

    def device_buffers(self):
        """Device pointers (bin, global, meta, out) of the handle's resident buffers."""
        ptrs = [ctypes.c_void_p() for _ in range(4)]
        _check(lib().kg_handle_device_buffers(self._h, *[ctypes.byref(p) for p in ptrs]))
        return tuple(p.value for p in ptrs)

    def run(self, n: int, out: np.ndarray = None):
        """Forward pass on the inputs already in the device buffers; reads back into `out` when given."""
        if out is not None and (out.dtype != np.float32 or not out.flags.c_contiguous or
                                out.size < n * self.net.row_len):
            raise ValueError(f"out must be contiguous float32 with room for {n} rows of {self.net.row_len}")
        _check(lib().kg_run(self._h, n, _ptr(out)))

    def featurize(self, positions, symmetry=None):
        """The device featurizer (kg_featurize) into the handle's device input buffers, without waiting."""
        sym = None if symmetry is None else np.ascontiguousarray(symmetry, np.int32)
        _check(lib().kg_featurize(self._h, len(positions), positions, _ptr(sym)))

    def run_static(self, n: int):
        """The allocation-free forward pass (kg_run_static): inputs in the device buffers, outputs left in the
        device output buffer, enqueued without waiting."""
        _check(lib().kg_run_static(self._h, n))

    def sync(self):
        _check(lib().kg_sync(self._h))

    @property
    def stream(self) -> int:
        return lib().kg_handle_stream(self._h)

    def _rows(self, rows, want_ownership):
        """Row inputs and output structures of get_output; `keep` holds the arrays they point into."""
        n = len(rows)
        keep = []
        arr = (RowInput * n)()
        outs = (NNOutput * n)()
        owners = []
        net = self.net
        for i, r in enumerate(rows):
            sp = np.ascontiguousarray(r["spatial"], np.float32)
            gl = np.ascontiguousarray(r["glob"], np.float32)
            me = r.get("meta")
            me = None if me is None else np.ascontiguousarray(me, np.float32)
            if sp.shape != (net.num_input_channels, 19, 19) or gl.shape != (net.num_global,):
                raise ValueError(f"row {i}: spatial must be [{net.num_input_channels}, 19, 19] and glob "
                                 f"[{net.num_global}], got {sp.shape} and {gl.shape}")
            if me is not None and me.shape != (net.num_meta,):
                raise ValueError(f"row {i}: meta must be [{net.num_meta}], got {me.shape}")
            keep += [sp, gl, me]
            arr[i].row_spatial = _ptr(sp).value
            arr[i].row_global = _ptr(gl).value
            arr[i].row_meta = None if me is None else _ptr(me).value
            arr[i].symmetry = int(r.get("symmetry", 0))
            arr[i].policy_optimism = float(r.get("policy_optimism", 0.0))
            own = np.zeros(HW, np.float32) if want_ownership else None
            owners.append(own)
            outs[i].white_owner_map = None if own is None else _ptr(own).value
        return arr, outs, owners, keep

    def get_output(self, rows, want_ownership=True):
        """NeuralNet::get_output. rows: list of dicts with spatial [C,19,19], glob [G], meta [192] or None,
        symmetry, policy_optimism. Returns a list of dicts of NNOutput fields."""
        arr, outs, owners, _keep = self._rows(rows, want_ownership)
        _check(lib().kg_get_output(self._h, len(rows), arr, outs))
        return [_output_dict(outs[i], owners[i]) for i in range(len(rows))]

    @staticmethod
    def _post(post, n):
        """post: one dict per row with legal [362] (bool), white_to_move, board_x_size, board_y_size, and optional
        nn_policy_temperature (1.0), enable_passing_hacks (False), no_result_allowed (True)."""
        if len(post) != n:
            raise ValueError(f"need {n} post-processing rows, got {len(post)}")
        arr = (PostInput * n)()
        keep = []
        for i, q in enumerate(post):
            legal = np.ascontiguousarray(q["legal"], np.uint8)
            if legal.shape != (MAX_POLICY,):
                raise ValueError(f"legal must be [{MAX_POLICY}], got {legal.shape}")
            keep.append(legal)
            arr[i].legal = _ptr(legal).value
            arr[i].white_to_move = int(bool(q["white_to_move"]))
            arr[i].board_x_size = int(q.get("board_x_size", 19))
            arr[i].board_y_size = int(q.get("board_y_size", 19))
            arr[i].nn_policy_temperature = float(q.get("nn_policy_temperature", 1.0))
            arr[i].enable_passing_hacks = int(bool(q.get("enable_passing_hacks", False)))
            arr[i].no_result_allowed = int(bool(q.get("no_result_allowed", True)))
        return arr, keep

    def get_output_eval(self, rows, post, want_ownership=True):
        """get_output followed by NNEvaluator's post-processing, on the device (kg_get_output_eval)."""
        arr, outs, owners, _keep = self._rows(rows, want_ownership)
        parr, _pkeep = self._post(post, len(rows))
        _check(lib().kg_get_output_eval(self._h, len(rows), arr, parr, outs))
        return [_output_dict(outs[i], owners[i]) for i in range(len(rows))]

    def evaluate_positions(self, positions, symmetry, policy_optimism, post, want_ownership=True):
        """Featurizer, forward pass and NNEvaluator's post-processing, all on the device (kg_evaluate_positions):
        positions from make_positions, one symmetry and policy optimism per row, post as in get_output_eval."""
        n = len(positions)
        sym = np.ascontiguousarray(np.broadcast_to(symmetry, (n,)), np.int32)
        opt = np.ascontiguousarray(np.broadcast_to(policy_optimism, (n,)), np.float32)
        parr, _pkeep = self._post(post, n)
        outs = (NNOutput * n)()
        owners = [np.zeros(HW, np.float32) if want_ownership else None for _ in range(n)]
        for i in range(n):
            outs[i].white_owner_map = None if owners[i] is None else _ptr(owners[i]).value
        _check(lib().kg_evaluate_positions(self._h, n, positions, _ptr(sym), _ptr(opt), parr, outs))
        return [_output_dict(outs[i], owners[i]) for i in range(n)]

    def post_outputs(self, raw, symmetry, policy_optimism, post, want_ownership=True):
        """copy_outputs and NNEvaluator's post-processing of raw rows given on the host, on the device
        (kg_post_outputs)."""
        raw = np.ascontiguousarray(raw, np.float32)
        n = raw.shape[0]
        if raw.shape != (n, self.net.row_len):
            raise ValueError(f"raw rows must be [n, {self.net.row_len}], got {raw.shape}")
        sym = np.ascontiguousarray(np.broadcast_to(symmetry, (n,)), np.int32)
        opt = np.ascontiguousarray(np.broadcast_to(policy_optimism, (n,)), np.float32)
        parr, _pkeep = self._post(post, n)
        outs = (NNOutput * n)()
        owners = [np.zeros(HW, np.float32) if want_ownership else None for _ in range(n)]
        for i in range(n):
            outs[i].white_owner_map = None if owners[i] is None else _ptr(owners[i]).value
        _check(lib().kg_post_outputs(self._h, n, _ptr(raw), _ptr(sym), _ptr(opt), parr, outs))
        return [_output_dict(outs[i], owners[i]) for i in range(n)]

    def get_output_async(self, rows, want_ownership=True, done=None):
        """get_output with the readback on the library's helper thread: returns once the batch is enqueued.
        `done(status)`, if given, is called from that thread. Returns a pending result whose wait() joins it
        (kg_wait) and gives the list of dicts of NNOutput fields."""
        arr, outs, owners, keep = self._rows(rows, want_ownership)
        cb = DONE_FN((lambda user, status: done(status)) if done else (lambda user, status: None))
        _check(lib().kg_get_output_async(self._h, len(rows), arr, outs, cb, None))
        handle = self

        class Pending:
            def wait(self_inner):
                _check(lib().kg_wait(handle._h))
                self_inner._keep = (arr, keep, cb)
                return [_output_dict(outs[i], owners[i]) for i in range(len(owners))]

        p = Pending()
        p._keep = (arr, outs, owners, keep, cb)  # alive until the helper thread has written the outputs
        return p

    def wait(self):
        _check(lib().kg_wait(self._h))

    # --- kernel timing ---
    def profile(self, enable: bool):
        _check(lib().kg_profile_enable(self._h, int(enable)))

    def profile_reset(self):
        _check(lib().kg_profile_reset(self._h))

    def profile_read(self):
        k = 32
        names = (ctypes.c_char_p * k)()
        launches = (ctypes.c_long * k)()
        ms = (ctypes.c_double * k)()
        flops = (ctypes.c_double * k)()
        byts = (ctypes.c_double * k)()
        n = lib().kg_profile_read(self._h, names, launches, ms, flops, byts, k)
        if n < 0:
            raise KgError("kg_profile_read failed")
        return {names[i].decode(): {"launches": launches[i], "ms": ms[i], "flops": flops[i], "bytes": byts[i]}
                for i in range(min(n, k))}

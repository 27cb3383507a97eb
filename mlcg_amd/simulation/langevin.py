"""BAOAB Langevin dynamics (mlcg/simulation/langevin.py, base.py).

``LangevinSimulation`` keeps the reference's constructor arguments that shape
the dynamics (``friction``, ``dt``, ``n_timesteps``, ``save_interval``,
``random_seed``, ``save_forces``, ``save_energies``, ``dtype``, ``compile``,
``compile_mode``, ``force_compile``) and its
``attach_model_and_configurations(model, configurations, beta)`` /
``simulate()`` / ``compile_model(data)`` entry points.  One timestep is

    BAOA kernel (mlcg_langevin_baoa)  ->  model forces  ->  B kernel

with the noise drawn in the kernel from a counter-based generator whose step
counter lives on the device, so the whole step -- including the radius-graph
rebuild at a fixed edge capacity -- can be captured once as a HIP graph and
replayed (``capture=True``).  The model is called exactly as the reference
calls it (``calculate_potential_and_forces``, base.py:517-539): a module whose
``forward(data)`` fills ``data.out["energy"]`` and ``data.out["forces"]``
(e.g. SumOut of GradientsOut models).

With ``filename`` set, the run is written as the reference writes it
(base.py:799-1040): every ``export_interval`` steps the saved frames go to
``{filename}_coords_{kkkk}.npy`` ([n_sims, export_interval / save_interval,
n_atoms, 3]; ``_forces_``/``_potential_`` likewise when asked), with
``create_checkpoints`` the current positions and velocities and the number
of files written go to ``{filename}_checkpoint.pt``, and ``log_interval``
logs progress by ``print`` or to ``{filename}_log.txt``.  A run started with
``read_checkpoint_file`` (True for ``{filename}_checkpoint.pt``, or a path)
continues from the checkpointed state and file index up to n_timesteps;
because the noise is a function of the step counter, the continued
trajectory is bit-identical to an uninterrupted run.  Parallel tempering
(parallel_tempering.py) is not part of this module.
"""

from __future__ import annotations

import math
import os
import time
import warnings
from typing import List, Optional, Union

import numpy as np
import torch

from .. import ops
from ..data import AtomicData
from ..data._keys import ENERGY_KEY, FORCE_KEY, MASS_KEY, POSITIONS_KEY, VELOCITY_KEY
from ..data.atomic_data import collate


def sample_maxwell_boltzmann(betas: torch.Tensor, masses: torch.Tensor,
                             generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """[N, 3] velocities with per-component variance 1/(beta m)
    (langevin.py:79-98)."""
    assert bool((masses > 0).all())
    scale = torch.sqrt(1.0 / (betas * masses))
    z = torch.randn(masses.shape[0], 3, generator=generator, dtype=masses.dtype)
    return z * scale[:, None]


class LangevinSimulation:
    def __init__(self, friction: float = 1e-3, dt: float = 5e-4, n_timesteps: int = 100,
                 save_interval: int = 10, random_seed: Optional[int] = None,
                 device: str = "cuda", dtype: str = "single", save_forces: bool = False,
                 save_energies: bool = False, capture: bool = False,
                 edge_capacity_factor: float = 1.5, check_interval: int = 100,
                 filename: Optional[str] = None, export_interval: Optional[int] = None,
                 log_interval: Optional[int] = None, log_type: str = "write",
                 create_checkpoints: bool = False,
                 read_checkpoint_file: Union[str, bool, None] = None,
                 compile: bool = False, compile_mode: str = "default",
                 force_compile: bool = False):
        assert friction > 0
        if dtype not in ("single", "double"):
            raise ValueError(f"dtype must be 'single' or 'double', got {dtype!r}")
        if dtype == "double" and capture:
            # the float64 model runs module by module: its radius graph is sized
            # on the host every step, which a captured graph cannot do
            raise ValueError("capture=True needs dtype='single'")
        if compile and capture:
            # the captured step already replays the kernels without the host;
            # torch.compile is for the eager loop
            raise ValueError("compile=True and capture=True are exclusive")
        if compile and compile_mode in ("reduce-overhead", "max-autotune"):
            # these modes record the model into CUDA graphs with torch's
            # cudagraph trees, which reject the device caches the HIP passes
            # build on first use (weight images, interaction structures)
            raise ValueError(
                f"compile_mode={compile_mode!r} records CUDA graphs through torch's cudagraph "
                "trees, which do not hold this library's device caches: use capture=True (the "
                "whole step as one HIP graph) or a mode without graphs ('default', "
                "'max-autotune-no-cudagraphs')")
        if n_timesteps % save_interval != 0:
            raise ValueError("n_timesteps must be a multiple of save_interval")
        self.friction = friction
        self.dt = dt
        self.n_timesteps = n_timesteps
        self.save_interval = save_interval
        self.random_seed = 0 if random_seed is None else int(random_seed)
        self.device = torch.device(device)
        self.dtype = torch.float64 if dtype == "double" else torch.float32
        self.save_forces = save_forces
        self.save_energies = save_energies
        self.capture = capture
        self.edge_capacity_factor = edge_capacity_factor
        self.check_interval = check_interval
        self.vscale = float(np.exp(-self.dt * self.friction))
        self.noisescale = float(np.sqrt(1 - self.vscale * self.vscale))
        self.model = None
        self.initial_data = None
        # export / log / checkpoint options (base.py:147-240, 629-720)
        self.filename = filename
        self.export_interval = n_timesteps if export_interval is None else int(export_interval)
        if self.export_interval % save_interval != 0:
            raise ValueError("export_interval must be a multiple of save_interval")
        if n_timesteps % self.export_interval != 0:
            raise ValueError("n_timesteps must be a multiple of export_interval")
        if log_type not in ("print", "write"):
            raise ValueError("log_type must be 'print' or 'write'")
        if filename is None and (export_interval is not None or create_checkpoints
                                 or (log_interval is not None and log_type == "write")):
            raise ValueError("filename is required for exports, checkpoints and written logs")
        self.log_interval = log_interval
        self.log_type = log_type
        self.create_checkpoints = create_checkpoints
        self.read_checkpoint_file = None if read_checkpoint_file is False else read_checkpoint_file
        self.current_timestep = 0  # files already written (restored from a checkpoint)
        # torch.compile of the model at the start of simulate() (base.py:447-489)
        self.compile = bool(compile)
        self.compile_mode = compile_mode
        self.force_compile = bool(force_compile)
        # hook run eagerly every `_hook_interval` steps on (x, v, F, potential)
        self._hook = None
        self._hook_interval = 0

    # ------------------------------------------------------------------
    def attach_model_and_configurations(self, model: torch.nn.Module,
                                        configurations: List[AtomicData],
                                        beta: Union[float, List[float]]):
        # the whole model in the simulation's precision (base.py:271): in
        # double, SchNet runs module by module in float64 (HIP gather, torch
        # linears) and the priors and the integrator use their float64 kernels
        self.model = model.eval().to(device=self.device, dtype=self.dtype)
        for p in self.model.parameters():
            p.requires_grad = False
        self._attach_configurations(configurations, beta)

    def _attach_configurations(self, configurations, beta):
        if len(configurations) == 0:
            raise ValueError("no configurations")
        n0 = configurations[0].pos.shape[0]
        for k, d in enumerate(configurations):
            if MASS_KEY not in d:
                raise ValueError(f"configuration {k} has no masses")
            if d.pos.shape != (n0, 3) or d.masses.shape != (n0,):
                raise ValueError(f"configuration {k} differs in shape from the first one")
        data = collate(configurations).to(self.device)
        data.pos = data.pos.to(self.dtype).contiguous()
        data.masses = data.masses.to(self.dtype).contiguous()
        self.n_sims = len(configurations)
        self.n_atoms = n0
        if isinstance(beta, (float, int)):
            if beta <= 0:
                raise ValueError(f"Beta must be positive, but {beta} was supplied")
            self.beta = torch.full((self.n_sims,), float(beta), dtype=self.dtype)
        else:
            self.beta = torch.tensor(beta, dtype=self.dtype)
            if not bool((self.beta > 0).all()):
                raise ValueError(f"All betas must be positive, but {beta} contains an "
                                 "illegal value.")
        assert len(self.beta) == self.n_sims
        betas = self.beta.repeat_interleave(self.n_atoms)
        if VELOCITY_KEY not in data:
            g = torch.Generator().manual_seed(self.random_seed)
            data[VELOCITY_KEY] = sample_maxwell_boltzmann(
                betas, data.masses.cpu(), generator=g).to(self.device, self.dtype)
        data[VELOCITY_KEY] = data[VELOCITY_KEY].to(self.device, self.dtype).contiguous()
        self.beta_mass_ratio = torch.sqrt(1.0 / betas.to(self.device) / data.masses).contiguous()
        if self.read_checkpoint_file is not None:
            self._read_checkpoint(data)
        self.initial_data = data

    def _checkpoint_path(self) -> str:
        if isinstance(self.read_checkpoint_file, str):
            return self.read_checkpoint_file
        if self.filename is None:
            raise ValueError("read_checkpoint_file=True needs a filename")
        return f"{self.filename}_checkpoint.pt"

    def _read_checkpoint(self, data):
        """Positions, velocities and the number of files written by an earlier
        run; its intervals win over the ones given here (base.py:653-695)."""
        path = self._checkpoint_path()
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} does not exist")
        ck = torch.load(path, map_location="cpu", weights_only=True)
        for key in ("export_interval", "save_interval", "log_interval"):
            if key in ck and ck[key] != getattr(self, key):
                warnings.warn(f"specified {key} doesn't match the checkpoint, using "
                              f"the checkpointed {key} instead", UserWarning)
                setattr(self, key, ck[key])
        if ck[POSITIONS_KEY].shape != data.pos.shape:
            raise ValueError("checkpoint positions do not match the configurations")
        data.pos = ck[POSITIONS_KEY].to(self.device, self.dtype).contiguous()
        data[VELOCITY_KEY] = ck[VELOCITY_KEY].to(self.device, self.dtype).contiguous()
        self.current_timestep = int(ck["current_timestep"])

    def _log(self, msg: str):
        if self.log_type == "print":
            print(msg, flush=True)
        else:
            with open(f"{self.filename}_log.txt", "a") as fh:
                fh.write(msg + "\n")

    def _export(self, index: int, coords, potential, forces, x, v):
        """Writes one export chunk ([n_sims, frames, n_atoms, 3] arrays) and,
        when asked, the checkpoint (base.py:930-990)."""
        key = f"{index:04d}"
        shape = (coords.shape[0], self.n_sims, self.n_atoms, 3)
        np.save(f"{self.filename}_coords_{key}.npy",
                coords.view(shape).permute(1, 0, 2, 3).cpu().numpy())
        if forces is not None:
            np.save(f"{self.filename}_forces_{key}.npy",
                    forces.view(shape).permute(1, 0, 2, 3).cpu().numpy())
        if potential is not None:
            np.save(f"{self.filename}_potential_{key}.npy", potential.t().cpu().numpy())
        if self.create_checkpoints:
            torch.save({POSITIONS_KEY: x.detach().cpu().clone(),
                        VELOCITY_KEY: v.detach().cpu().clone(),
                        "current_timestep": index + 1,
                        "export_interval": self.export_interval,
                        "save_interval": self.save_interval,
                        "log_interval": self.log_interval},
                       f"{self.filename}_checkpoint.pt")

    # ------------------------------------------------------------------
    def calculate_potential_and_forces(self, data):
        # grad mode on, as the reference's loop runs: a model without a fused
        # pass (a float64 model runs module by module) gets its forces from
        # GradientsOut's autograd; the fused passes record nothing, since the
        # parameters do not require gradients
        with torch.enable_grad():
            data = self.model(data)
        return data.out[ENERGY_KEY].detach(), data.out[FORCE_KEY].detach()

    def _run_and_check(self, data):
        """One model call whose energies and forces must be finite
        (base.py:434-445)."""
        potential, forces = self.calculate_potential_and_forces(data)
        if not bool(torch.isfinite(forces).all()):
            raise RuntimeError("Invalid values detected in computed forces.")
        if not bool(torch.isfinite(potential).all()):
            raise RuntimeError("Invalid values detected in computed potential.")

    def compile_model(self, data):
        """With ``compile=True``: ``torch.compile(model, dynamic=True,
        mode=compile_mode)`` (base.py:447-489).  A batch of one structure is
        left eager unless ``force_compile``; if compiling or the first
        compiled call fails, the model is compiled again with dynamo's
        suppress_errors, so the failing parts run eagerly.  Either way the
        model is run once and its outputs checked for non-finite values.

        The fused SchNet and prior passes launch HIP kernels through ctypes,
        so dynamo runs them as opaque calls (graph breaks); the compiler
        works on the torch code around them."""
        if self.compile:
            if int(data.batch.max()) == 0 and not self.force_compile:
                warnings.warn(
                    "Compilation is allowed only when more than one structure is provided; "
                    "the simulation runs in non-compiled mode (force_compile=True overrides "
                    "this, with the risks of compiled scatter operations on one structure)")
            else:
                if int(data.batch.max()) == 0:
                    warnings.warn("Forcing compilation with only one structure in the batch")
                import logging
                import torch._dynamo

                torch._logging.set_logs(dynamo=logging.ERROR)
                try:
                    self.model = torch.compile(self.model, dynamic=True, mode=self.compile_mode)
                    self._run_and_check(data)
                    return
                except Exception as e:  # the reference's fallback, base.py:467-486
                    warnings.warn(f"torch.compile failed ({e}); compiling again with "
                                  "torch._dynamo.config.suppress_errors = True")
                    torch._dynamo.config.suppress_errors = True
                    model = getattr(self.model, "_orig_mod", self.model)
                    self.model = torch.compile(model, dynamic=True, mode=self.compile_mode)
        self._run_and_check(data)

    def _set_capacity(self, data):
        """Fixed radius-graph capacities for every SchNet in the model (from
        the initial structure's edge count), so that no step synchronises."""
        from ..nn.schnet import SchNet

        for m in self.model.modules():
            if isinstance(m, SchNet) and m.graph_capacity is None and m.fused_spec() is not None:
                g = m.build_graph(data)
                cap = int(math.ceil(g.num_edges * self.edge_capacity_factor)) + 64
                m.graph_capacity = cap + (cap % 2)

    def _graph_flags(self):
        from ..nn.schnet import SchNet

        return [m.last_graph.flags for m in self.model.modules()
                if isinstance(m, SchNet) and m.last_graph is not None
                and m.graph_capacity is not None]

    def _check_flags(self, sticky):
        """Raises if any step since the start of the run overflowed a radius
        graph: `sticky` is the OR of every step's graph flags, accumulated on
        the device inside the (captured) step, so an overflow between two
        checks is not lost."""
        from .. import ops

        ops.check_numerics(self.device)
        v = int(sticky.item())
        if v:
            ops.radius_flags_read(v)
            if v & 8:  # a look-back timed out: the captured step's workspaces restart
                for ws in getattr(self, "_radius_ws", []):
                    ws.zero_()
            hint = ("raise edge_capacity_factor or max_num_neighbors" if v & 3
                    else "an internal failure of the radius kernel")
            raise RuntimeError(
                f"radius graph overflow flags {v} ({ops.radius_flags_message(v)}) in a step before "
                f"step {self.current_step_for_check}: {hint}")

    def simulate(self) -> np.ndarray:
        """Runs the BAOAB steps up to n_timesteps (from the checkpointed step
        when resuming); returns the saved positions [n_sims, n_saves, n_atoms,
        3] -- with a filename, those of the last export chunk -- and stores
        energies/forces if asked."""
        if self.model is None or self.initial_data is None:
            raise RuntimeError("attach a model and configurations first")
        data = self.initial_data.clone()
        x, v, m = data.pos, data.velocities.contiguous(), data.masses
        data.velocities = v
        self._set_capacity(data)
        # resumed runs continue the step counter, hence the noise stream
        t_init = self.current_timestep * self.export_interval
        step_ctr = torch.full((1,), t_init, dtype=torch.int64, device=self.device)
        epot = torch.zeros(self.n_sims, dtype=self.dtype, device=self.device)
        F = torch.zeros_like(x)
        # OR of the radius-graph flags of every step (bit 0: max_num_neighbors
        # bound, bit 1: edge capacity exceeded); read only at the checks
        sticky = torch.zeros(1, dtype=torch.int32, device=self.device)

        def or_flags():
            for fl in self._graph_flags():
                sticky.bitwise_or_(fl)

        with torch.no_grad():
            self.compile_model(data)
            e0, f0 = self.calculate_potential_and_forces(data)
            or_flags()
        F.copy_(f0)
        epot.copy_(e0)
        # frames held on the device: one export chunk when writing files, the
        # whole run otherwise
        n_saves = (self.export_interval if self.filename is not None
                   else self.n_timesteps) // self.save_interval
        traj = torch.empty(n_saves, *x.shape, dtype=self.dtype, device=self.device)
        saved_e = (torch.empty(n_saves, self.n_sims, dtype=self.dtype, device=self.device)
                   if self.save_energies else None)
        saved_f = (torch.empty(n_saves, *x.shape, dtype=self.dtype, device=self.device)
                   if self.save_forces else None)

        def one_step():
            ops.langevin_baoa(x, v, F, m, self.beta_mass_ratio, self.dt, self.vscale,
                              self.noisescale, self.random_seed, step=step_ctr)
            data.pos = x
            e, f = self.calculate_potential_and_forces(data)
            or_flags()
            if ops.copy_batch_ok([F, epot], [f, e]):
                ops.copy_batch([F, epot], [f, e])  # one launch for both
            else:
                F.copy_(f)
                epot.copy_(e)
            ops.langevin_b(v, F, m, self.dt, step=step_ctr)

        graph = None
        self.current_step_for_check = t_init
        if self.log_interval is not None:
            self._log(f"Generating {self.n_sims} simulations of n_timesteps {self.n_timesteps} "
                      f"saved at {self.save_interval}-step intervals ({time.asctime()})")
        # steady-state timing: steps after the capture (or after step 2)
        self.timed_steps = 0
        self.timed_seconds = 0.0
        t_start = None
        with torch.no_grad():
            for t in range(t_init, self.n_timesteps):
                if t == t_init + 3:
                    torch.cuda.synchronize()
                    t_start = time.perf_counter()
                self.current_step_for_check = t + 1
                if graph is None and self.capture and t >= t_init + 2:
                    torch.cuda.synchronize()
                    self._check_flags(sticky)
                    graph = torch.cuda.CUDAGraph()
                    # the step's radius-graph workspaces, zero-filled once
                    # here rather than by a fill every replay would rerun
                    self._radius_ws = ops.reserve_radius_workspaces(
                        x.shape[0], x.device, len(self._graph_flags()) or 1)
                    torch.cuda.synchronize()
                    try:
                        with torch.cuda.graph(graph):
                            one_step()
                    finally:
                        ops.release_radius_workspaces(x.device)
                    graph.replay()  # the captured step is step t
                elif graph is not None:
                    graph.replay()
                else:
                    one_step()
                if self._hook is not None and (t + 1) % self._hook_interval == 0:
                    self._hook(x, v, F, epot)
                if (t + 1) % self.save_interval == 0:
                    k = ((t + 1) // self.save_interval - 1) % n_saves
                    traj[k].copy_(x)
                    if saved_e is not None:
                        saved_e[k].copy_(epot)
                    if saved_f is not None:
                        saved_f[k].copy_(F)
                if (t + 1) % self.check_interval == 0:
                    self._check_flags(sticky)
                    if not bool(torch.isfinite(x).all()):
                        raise RuntimeError(f"non-finite positions at step {t + 1}")
                if self.filename is not None and (t + 1) % self.export_interval == 0:
                    self._check_flags(sticky)
                    self._export((t + 1) // self.export_interval - 1, traj, saved_e, saved_f,
                                 x, v)
                if self.log_interval is not None and (t + 1) % self.log_interval == 0:
                    self._log(f"{(t + 1) // self.save_interval} / "
                              f"{self.n_timesteps // self.save_interval} time points saved "
                              f"({time.asctime()})")
        torch.cuda.synchronize()
        if t_start is not None:
            self.timed_seconds = time.perf_counter() - t_start
            self.timed_steps = self.n_timesteps - t_init - 3
        self._check_flags(sticky)
        self.final_data = data
        self.potential = epot
        self.forces = F
        shape = (n_saves, self.n_sims, self.n_atoms, 3)
        out = traj.view(shape).permute(1, 0, 2, 3).cpu().numpy()
        self.simulated_coords = out
        if saved_e is not None:
            self.simulated_potential = saved_e.t().cpu().numpy()
        if saved_f is not None:
            self.simulated_forces = saved_f.view(shape).permute(1, 0, 2, 3).cpu().numpy()
        return out

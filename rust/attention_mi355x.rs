//! `--attention-backend mi355x`: paged decode and ragged / paged causal prefill on the
//! gfx950 kernels of `libmi355x_attn.so`, through the raw ABI of the `mi355x_sys` crate.
//!
//! Drop-in for the reference server: this file becomes `src/models/attention/mi355x.rs`, a
//! child module of `backend.rs` (so it sees the private `AttentionBackend` trait,
//! `backend.rs:262-306`), declared there with `#[cfg(has_mi355x)] mod mi355x;`. It keeps the
//! trait's contract (one plan per forward, reused by every layer; graph plans re-made
//! outside capture at a fixed address; the decode/prefill routing of `forward`) and the
//! reference's error strings, so callers see the same behaviour.
//!
//! Plan lifetime is this module's own: every native plan lives in a `PlanOwner`, which
//! knows which `*_plan_drop` entry frees it and carries two flags. `leased` is set while a
//! batch holds the backend's decode or prefill plan (a `Mi355xLease`; re-planning it then
//! fails, since the batch's layers still read it). `retired` is set when the decode graph
//! that registered a graph plan is dropped; retired graph plans leave the registry at the
//! next lookup, and the native plan is freed when its last holder lets go.
//!
//! No output tensor is allocated by the library: decode and prefill write into a tensor
//! allocated here (or the caller's static output in `forward_into`).

use std::{
    cell::{Cell, RefCell},
    ffi::c_void,
    rc::Rc,
};

use mi355x_sys as sys;
use tch::{Device, Kind, Tensor};

use crate::engine::{
    AttentionMetadata, BatchPhase, DecodeGraphState, DecodeHostMetadata, MetadataRequirements,
};

use super::{
    AttentionBackend, AttentionSpec, BackendPlan, BaseAttention, FlashAttentionBackend,
    PrefillMetadata, Result, model_error,
};

/// Which native planner made a plan; selects the entry that frees it.
#[derive(Clone, Copy, PartialEq, Eq)]
enum PlanKind {
    Decode,
    Prefill,
}

/// One native plan handle (null until the first prepare) and its lease state.
pub(super) struct PlanOwner {
    kind: PlanKind,
    handle: Cell<*mut c_void>,
    /// KV page size of the last prepare (the run entries check it against the plan).
    page_size: Cell<i64>,
    /// A batch holds this plan; it must not be re-planned until the batch is dropped.
    leased: Cell<bool>,
    /// Graph plans only: the graph that registered it is gone.
    retired: Cell<bool>,
}

impl PlanOwner {
    fn new(kind: PlanKind) -> Rc<Self> {
        Rc::new(Self {
            kind,
            handle: Cell::new(std::ptr::null_mut()),
            page_size: Cell::new(0),
            leased: Cell::new(false),
            retired: Cell::new(false),
        })
    }

    /// Runs a native prepare on this owner's handle (null makes a new plan) and keeps the
    /// handle it returns. The native planners re-plan an existing handle in place.
    fn replan(
        &self,
        page_size: i64,
        prepare: impl FnOnce(*mut c_void) -> Result<*mut c_void>,
    ) -> Result<()> {
        let before = self.handle.get();
        let after = prepare(before)?;
        if !before.is_null() && after != before {
            return Err(model_error("graph plan address changed"));
        }
        self.handle.set(after);
        self.page_size.set(page_size);
        Ok(())
    }
}

impl Drop for PlanOwner {
    fn drop(&mut self) {
        let handle = self.handle.get();
        if handle.is_null() {
            return;
        }
        // The library waits for the plan's pending uploads before freeing it.
        unsafe {
            match self.kind {
                PlanKind::Decode => sys::mi355x_decode_plan_drop(handle),
                PlanKind::Prefill => sys::mi355x_prefill_plan_drop(handle),
            }
        }
    }
}

/// A batch's hold on a plan, carried in `BackendPlan::Mi355x{Decode,Prefill}`. An
/// exclusive lease (the backend's per-forward plans) clears `leased` when dropped; a graph
/// plan is shared by every replay and is never leased exclusively.
pub(super) struct Mi355xLease {
    owner: Rc<PlanOwner>,
    exclusive: bool,
}

impl Mi355xLease {
    fn exclusive(owner: &Rc<PlanOwner>, busy: &str) -> Result<Self> {
        if owner.leased.replace(true) {
            return Err(model_error(busy));
        }
        Ok(Self {
            owner: Rc::clone(owner),
            exclusive: true,
        })
    }

    fn shared(owner: &Rc<PlanOwner>) -> Self {
        Self {
            owner: Rc::clone(owner),
            exclusive: false,
        }
    }

    fn handle(&self) -> *mut c_void {
        self.owner.handle.get()
    }

    fn page_size(&self) -> i64 {
        self.owner.page_size.get()
    }
}

impl Drop for Mi355xLease {
    fn drop(&mut self) {
        if self.exclusive {
            self.owner.leased.set(false);
        }
    }
}

/// Graph plans of the live decode graphs, found by the address of the block table the
/// graph was captured on (a handful of batch buckets, so a short list).
#[derive(Default)]
struct GraphPlans(Vec<(usize, Rc<PlanOwner>)>);

impl GraphPlans {
    fn prune(&mut self) {
        self.0.retain(|(_, owner)| !owner.retired.get());
    }

    fn find(&self, table_addr: usize) -> Option<&Rc<PlanOwner>> {
        self.0
            .iter()
            .find(|(addr, owner)| *addr == table_addr && !owner.retired.get())
            .map(|(_, owner)| owner)
    }
}

pub(super) struct Mi355xAttentionBackend {
    decode: Rc<PlanOwner>,
    prefill: Rc<PlanOwner>,
    graphs: RefCell<GraphPlans>,
}

impl Default for Mi355xAttentionBackend {
    fn default() -> Self {
        Self {
            decode: PlanOwner::new(PlanKind::Decode),
            prefill: PlanOwner::new(PlanKind::Prefill),
            graphs: RefCell::new(GraphPlans::default()),
        }
    }
}

fn dtype_code(kind: Kind) -> Result<i64> {
    match kind {
        Kind::BFloat16 => Ok(0),
        Kind::Half => Ok(1),
        _ => Err(model_error("mi355x attention requires bfloat16 or float16")),
    }
}

fn stream_of(device: Device) -> *mut c_void {
    match device {
        Device::Cuda(index) => sys::current_stream(index as i64),
        _ => std::ptr::null_mut(),
    }
}

fn check(status: *const std::ffi::c_char, what: &str) -> Result<()> {
    sys::check(status).map_err(|error| model_error(&format!("{what}: {error}")))
}

fn bound_page_size(page_size: Option<i64>) -> Result<i64> {
    page_size.ok_or_else(|| model_error("mi355x requires a bound KV cache"))
}

impl AttentionBackend for Mi355xAttentionBackend {
    fn metadata_requirements(&self, _phase: BatchPhase) -> MetadataRequirements {
        MetadataRequirements {
            block_table: true,
            req_to_token: false,
        }
    }

    fn supports_cuda_graph(&self) -> bool {
        true
    }

    fn prepare_decode_graph(
        &self,
        metadata: &AttentionMetadata,
        spec: AttentionSpec,
        page_size: i64,
    ) -> Result<Option<Box<dyn DecodeGraphState>>> {
        let (Some(table), Some(lengths)) = (&metadata.block_table, &metadata.cache_seqlens) else {
            return Err(model_error(if metadata.block_table.is_none() {
                "missing graph block_table"
            } else {
                "missing graph cache_seqlens"
            }));
        };
        let mut graphs = self.graphs.borrow_mut();
        graphs.prune();
        let addr = table.data_ptr() as usize;
        if graphs.find(addr).is_some() {
            return Err(model_error("decode graph buffers are already registered"));
        }
        let owner = PlanOwner::new(PlanKind::Decode);
        owner.replan(page_size, |existing| {
            prepare_decode(metadata, spec, page_size, existing, true)
        })?;
        graphs.0.push((addr, Rc::clone(&owner)));
        Ok(Some(Box::new(Mi355xGraphState {
            owner,
            table: table.shallow_clone(),
            lengths: lengths.shallow_clone(),
            spec,
        })))
    }

    fn prepare(
        &self,
        metadata: Option<&AttentionMetadata>,
        prefill: &PrefillMetadata,
        spec: AttentionSpec,
        page_size: Option<i64>,
    ) -> Result<BackendPlan> {
        let Some(metadata) = metadata else {
            return FlashAttentionBackend.prepare(metadata, prefill, spec, page_size);
        };
        if metadata.forward_mode == BatchPhase::Decode {
            // A replayed graph's plan was re-made outside capture by `prepare_replay`: hand
            // it out as is (no device read-back, no allocation during capture).
            if let Some(table) = &metadata.block_table {
                if let Some(owner) = self.graphs.borrow().find(table.data_ptr() as usize) {
                    return Ok(BackendPlan::Mi355xDecode(Mi355xLease::shared(owner)));
                }
            }
            let page_size = bound_page_size(page_size)?;
            let lease =
                Mi355xLease::exclusive(&self.decode, "previous mi355x batch is still in use")?;
            // On failure the lease drops here and frees the plan for the next attempt.
            self.decode.replan(page_size, |existing| {
                prepare_decode(metadata, spec, page_size, existing, false)
            })?;
            return Ok(BackendPlan::Mi355xDecode(lease));
        }
        let page_size = bound_page_size(page_size)?;
        let lease = Mi355xLease::exclusive(
            &self.prefill,
            "previous mi355x prefill batch is still in use",
        )?;
        self.prefill.replan(page_size, |existing| {
            prepare_prefill(metadata, prefill, spec, page_size, existing)
        })?;
        Ok(BackendPlan::Mi355xPrefill(lease, prefill.has_prefix()))
    }

    fn forward(
        &self,
        q: &Tensor,
        k: &Tensor,
        v: &Tensor,
        cache: &BaseAttention,
        prefill: &PrefillMetadata,
        metadata: Option<&AttentionMetadata>,
        num_heads: i64,
        num_kv_heads: i64,
        head_dim: i64,
        plan: &BackendPlan,
    ) -> Result<Tensor> {
        match metadata.map(|meta| meta.forward_mode) {
            Some(BatchPhase::Decode) => mi355x_decode(q, cache, plan, num_kv_heads, head_dim, None),
            Some(_) => mi355x_prefill(q, k, v, cache, plan, num_kv_heads, head_dim, None),
            None => FlashAttentionBackend.forward(
                q,
                k,
                v,
                cache,
                prefill,
                metadata,
                num_heads,
                num_kv_heads,
                head_dim,
                plan,
            ),
        }
    }
}

/// Decode graph state: the graph's own plan, sized for the captured bucket, re-made in
/// place before every replay. Dropping it retires the plan from the backend's registry.
struct Mi355xGraphState {
    owner: Rc<PlanOwner>,
    table: Tensor,
    lengths: Tensor,
    spec: AttentionSpec,
}

impl Drop for Mi355xGraphState {
    fn drop(&mut self) {
        self.owner.retired.set(true);
    }
}

impl DecodeGraphState for Mi355xGraphState {
    fn prepare_replay(&self, host: Option<&DecodeHostMetadata>) -> Result<()> {
        // The captured bucket has `rows` rows; rows past the live batch are pad rows that
        // read page 0 with length 1 (and write the reserved slot), so their host length is 1.
        let rows = self.table.size()[0] as usize;
        let decode_host = host.map(|host| {
            let live = host.cache_seqlens.len().min(rows);
            let mut cache_seqlens = Vec::with_capacity(rows);
            cache_seqlens.extend_from_slice(&host.cache_seqlens[..live]);
            cache_seqlens.extend(std::iter::repeat(1).take(rows - live));
            DecodeHostMetadata {
                cache_seqlens,
                block_table_versions: None,
            }
        });
        let metadata = AttentionMetadata {
            forward_mode: BatchPhase::Decode,
            decode_host,
            write_loc: None,
            cu_seqlens_q: None,
            prefix_lens: None,
            block_table: Some(self.table.shallow_clone()),
            cache_seqlens: Some(self.lengths.shallow_clone()),
            req_to_token: None,
            max_seqlen: None,
        };
        let page_size = self.owner.page_size.get();
        // `replan` refuses a handle that moved: the captured kernels hold its address.
        self.owner.replan(page_size, |existing| {
            prepare_decode(&metadata, self.spec, page_size, existing, true)
        })
    }

    fn needs_req_to_token(&self) -> bool {
        false
    }
}

/// `mi355x_decode_prepare` on the step's block table and lengths (the scheduler's host
/// lengths when present, so planning never reads the device back).
fn prepare_decode(
    metadata: &AttentionMetadata,
    spec: AttentionSpec,
    page_size: i64,
    existing: *mut c_void,
    graph: bool,
) -> Result<*mut c_void> {
    let table = metadata
        .block_table
        .as_ref()
        .ok_or_else(|| model_error("mi355x decode requires block_table"))?;
    let lengths = metadata
        .cache_seqlens
        .as_ref()
        .ok_or_else(|| model_error("mi355x decode requires cache_seqlens"))?;
    if table.dim() != 2 || table.kind() != Kind::Int || lengths.kind() != Kind::Int {
        return Err(model_error("invalid decode block table or lengths"));
    }
    let (rows, cols) = (table.size()[0], table.size()[1]);
    let (host_ptr, host_rows) = match &metadata.decode_host {
        Some(host) => (host.cache_seqlens.as_ptr(), host.cache_seqlens.len() as i64),
        None => (std::ptr::null(), 0),
    };
    let prepared = unsafe {
        sys::mi355x_decode_prepare(
            existing,
            table.data_ptr().cast(),
            rows,
            cols,
            table.stride()[0],
            lengths.data_ptr().cast(),
            spec.num_heads,
            spec.num_kv_heads,
            spec.head_dim,
            page_size,
            dtype_code(spec.kind)?,
            graph,
            host_ptr,
            host_rows,
            stream_of(spec.device),
        )
    };
    if prepared.is_null() {
        return Err(model_error(&format!(
            "mi355x decode plan failed: {}",
            sys::last_error()
        )));
    }
    Ok(prepared)
}

/// `mi355x_prefill_prepare` from the host snapshot `Attention::prepare` already took
/// (`PrefillMetadata`), so the plan needs no device read-back.
fn prepare_prefill(
    metadata: &AttentionMetadata,
    prefill: &PrefillMetadata,
    spec: AttentionSpec,
    page_size: i64,
    existing: *mut c_void,
) -> Result<*mut c_void> {
    let cumulative = metadata
        .cu_seqlens_q
        .as_ref()
        .ok_or_else(|| model_error("missing cu_seqlens_q"))?;
    let table = metadata.block_table.as_ref();
    if prefill.has_prefix() && table.is_none() {
        return Err(model_error("missing block_table"));
    }
    let boundaries: Vec<i32> = prefill.boundaries.iter().map(|&v| v as i32).collect();
    let prefixes: Vec<i32> = prefill.prefixes.iter().map(|&v| v as i32).collect();
    let (table_ptr, columns, stride) = match table {
        Some(t) => (t.data_ptr().cast_const().cast(), t.size()[1], t.stride()[0]),
        None => (std::ptr::null(), 0, 0),
    };
    let prepared = unsafe {
        sys::mi355x_prefill_prepare(
            existing,
            cumulative.data_ptr().cast(),
            table_ptr,
            prefixes.len() as i64,
            columns,
            stride,
            boundaries.as_ptr(),
            prefixes.as_ptr(),
            spec.num_heads,
            spec.num_kv_heads,
            page_size,
            dtype_code(spec.kind)?,
            stream_of(spec.device),
        )
    };
    if prepared.is_null() {
        return Err(model_error(&format!(
            "mi355x prefill plan failed: {}",
            sys::last_error()
        )));
    }
    Ok(prepared)
}

/// The output a run writes: the caller's static tensor, or a new [tokens, heads * 128].
fn output_for(q: &Tensor, head_dim: i64, output: Option<&Tensor>) -> Tensor {
    match output {
        Some(out) => out.shallow_clone(),
        None => Tensor::empty([q.size()[0], q.size()[1] * head_dim], (q.kind(), q.device())),
    }
}

/// Paged decode into `output` ([tokens, heads * 128], contiguous) or a new tensor. The
/// query may be a strided view of packed QKV (no contiguous copy, unlike
/// `backend.rs:651`).
pub(super) fn mi355x_decode(
    q: &Tensor,
    cache: &BaseAttention,
    plan: &BackendPlan,
    num_kv_heads: i64,
    head_dim: i64,
    output: Option<&Tensor>,
) -> Result<Tensor> {
    if !matches!(q.device(), Device::Cuda(_)) {
        return Err(model_error("mi355x decode requires a GPU device"));
    }
    let BackendPlan::Mi355xDecode(lease) = plan else {
        return Err(model_error("mi355x decode requires a prepared batch"));
    };
    let (k_cache, v_cache) = cache.cache_tensors()?;
    let out = output_for(q, head_dim, output);
    let (tokens, heads) = (q.size()[0], q.size()[1]);
    let qs = q.stride();
    check(
        unsafe {
            sys::mi355x_decode_run(
                lease.handle(),
                q.data_ptr().cast_const(),
                qs[0],
                qs[1],
                k_cache.data_ptr().cast_const(),
                v_cache.data_ptr().cast_const(),
                out.data_ptr(),
                heads * head_dim,
                head_dim,
                tokens,
                heads,
                num_kv_heads,
                lease.page_size(),
                dtype_code(q.kind())?,
                stream_of(q.device()),
            )
        },
        "mi355x decode failed",
    )?;
    Ok(out)
}

/// Ragged (no prefix) or paged (cached prefix) causal prefill, chosen once at prepare.
pub(super) fn mi355x_prefill(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    cache: &BaseAttention,
    plan: &BackendPlan,
    num_kv_heads: i64,
    head_dim: i64,
    output: Option<&Tensor>,
) -> Result<Tensor> {
    let BackendPlan::Mi355xPrefill(lease, paged) = plan else {
        return Err(model_error("missing mi355x prefill plan"));
    };
    // Paged plans read the layer's whole cache [pages, page, kv_heads, 128] (row stride
    // kv_heads * 128, head stride 128); ragged plans read the (packed) K/V projection rows
    // in place with their own strides.
    let (k_src, v_src, k_strides, v_strides) = if *paged {
        let (k_cache, v_cache) = cache.cache_tensors()?;
        let row = num_kv_heads * head_dim;
        (k_cache, v_cache, [row, head_dim], [row, head_dim])
    } else {
        let (ks, vs) = (k.stride(), v.stride());
        (k, v, [ks[0], ks[1]], [vs[0], vs[1]])
    };
    let out = output_for(q, head_dim, output);
    let (tokens, heads) = (q.size()[0], q.size()[1]);
    let qs = q.stride();
    check(
        unsafe {
            sys::mi355x_prefill_run(
                lease.handle(),
                q.data_ptr().cast_const(),
                qs[0],
                qs[1],
                k_src.data_ptr().cast_const(),
                k_strides[0],
                k_strides[1],
                v_src.data_ptr().cast_const(),
                v_strides[0],
                v_strides[1],
                out.data_ptr(),
                heads * head_dim,
                head_dim,
                tokens,
                heads,
                num_kv_heads,
                lease.page_size(),
                dtype_code(q.kind())?,
                stream_of(q.device()),
            )
        },
        "mi355x prefill failed",
    )?;
    Ok(out)
}
